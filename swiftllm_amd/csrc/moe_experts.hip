// MoE expert computation for gfx950: the grouped expert GEMM (with the
// SwiGLU gate fused into its epilogue) and the weighted combine.
//
// The reference names these steps in MoeMlp::forward
// (crates/swiftllm-models/src/layers/mlp.rs:240-246: "route tokens to
// experts", "combine expert outputs") over GatedMlp experts
// (mlp.rs:118-160: output = down_proj(silu(gate_proj(x)) * up_proj(x)),
// silu(x) = x / (1 + exp(-x)) at mlp.rs:263-265), with Linear weights laid
// out [out_features, in_features] (layers/mod.rs:22-24). All of it returns
// zeros in the reference.
//
// expert GEMM: the rows of `a` are expert-contiguous (the dispatch's x_perm:
//   expert e owns rows [offsets[e], offsets[e+1])). For each expert,
//   c[rows, :] = a[rows, :] . w[e]^T, or with a second weight (gated)
//   c = silu(a . w[e]^T) * (a . w2[e]^T). fp16 in, fp32 accumulate, fp16 out.
//   Workgroup tile 256 activation rows x 256 weight rows (plain: 256 output
//   columns; gated: 128 gate rows and their 128 up rows), k in steps of 64
//   (one 128-byte line of each row) copied from memory straight into two
//   LDS stages by buffer loads (128 KiB: one stage loads while the other is
//   multiplied; rows swizzled by 16-byte chunk so the operand reads are free
//   of bank conflicts); eight waves of 128 x 64,
//   each on v_mfma_f32_32x32x16_f16 with the weight as the MFMA's row
//   operand, so a lane ends with 4 consecutive output columns of one row
//   (8-byte stores) and, gated, holds the gate and up value of each of its
//   columns. The 256 x 256 tile does 128 FLOP per byte staged, so L2 feeds
//   the matrix cores at ~20 TB/s. Tiles are (expert, 256-row tile, column
//   tile); a workgroup finds its expert from the offsets, and the grid is
//   sized for the worst case (ceil(rows / 256) + E row tiles); surplus
//   workgroups exit at once.
// combine: out[t, :] = sum_k weights[t, k] * y[inverse[t, k], :] in fp32
//   (k ascending, fused multiply-add), rounded once to fp16; entries with
//   inverse -1 contribute nothing.

#include "common.hpp"

namespace swiftllm {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 256;        // activation rows per workgroup tile
constexpr int kBW = 256;        // weight rows per workgroup tile (gated: 128 gate + 128 up)
constexpr int kBK = 64;         // k per LDS stage: one 128-byte line of each tile row
constexpr int kKMult = 64;      // k must be a multiple of this (the API's contract)
constexpr int kMaxK = 1 << 21;  // k limit of the 32-bit buffer offsets
constexpr int kAStages = 2;     // LDS buffers of the activation tile: one stage in flight
constexpr int kWStages = 3;     // LDS buffers of the weight tile: two stages in flight
constexpr int kThreads = 512;   // 8 waves: 2 (rows) x 4 (weight rows), 128 x 64 each
constexpr int kRowChunks = kBK / 8;                        // 16-byte chunks per tile row
constexpr int kTileChunks = kBM * kRowChunks;              // chunks per operand tile
constexpr int kLoads = kTileChunks / kThreads;             // direct loads per thread per tile
constexpr size_t kTileHalfs = static_cast<size_t>(kBM) * kBK;  // one operand tile of a stage
static_assert(kBM == kBW, "activation and weight tiles share one LDS buffer size");
// LDS: activation buffers, then weight buffers, 32 KiB each: 160 KiB, all of
// a CU's LDS. The expert tile table sits in the last weight buffer until the
// main loop first writes there.
constexpr size_t kLdsHalfs = (kAStages + kWStages) * kTileHalfs;
constexpr int kMaxE = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kXcds = 8;                 // MI355X: 8 XCDs, each with its own L2
// Super-tiles per XCD: kSuper workgroups (one XCD's resident set) as
// super_m row tiles x kSuper / super_m column tiles. Measured on config 8:
// the gate and up GEMM ran 4% faster at 8 x 4 (or 16 x 2) than at 4 x 8 or
// 2 x 16; the down GEMM varies by about 1% over all shapes, fastest at
// 16 x 2. Shapes of more than 32 workgroups (16 x 4, 12 x 4) ran 10% slower.
constexpr int kSuperMGated = 8;
constexpr int kSuperMPlain = 16;
constexpr int kSuper = 32;
constexpr int kRsrcWord3 = 0x00020000;   // gfx9 buffer resource: raw 32-bit dwords

struct GemmArgs {
    const f16* a;        // [m_total][k]
    const f16* w;        // [E][n][k]
    const f16* w2;       // [E][n][k] or null
    const int* offsets;  // [E + 1]
    f16* c;              // [m_total][n]
    int E;
    int m_total;
    int n;
    int k;
    int m_tiles_max;     // row tiles the grid covers
    int n_tiles;         // column tiles
    int sm;              // super-tiles along the rows
    int super_m;         // row tiles per super-tile (column tiles: kSuper / super_m)
};

typedef __attribute__((address_space(3))) void* lds_ptr;
__device__ __forceinline__ lds_ptr to_lds(f16* p) { return (lds_ptr)p; }

__device__ __forceinline__ f16x mfma32(h8 a, h8 b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Output columns per workgroup tile: 256 plain, 128 gated (each column needs
// its gate and its up row).
template <bool GATED>
constexpr int tile_cols() { return GATED ? kBW / 2 : kBW; }

template <bool GATED>
__global__ __launch_bounds__(kThreads) void moe_expert_gemm_kernel(const GemmArgs a) {
    extern __shared__ __align__(16) f16 lds[];
    // First global row tile of each expert, in the last weight buffer (free
    // until the main loop loads its first stage there, after a barrier).
    int* s_tile0 = reinterpret_cast<int*>(lds + (kAStages + kWStages - 1) * kTileHalfs);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar LDS addresses

    // Which (row tile, column tile). Workgroups go to the 8 XCDs round
    // robin, so slot = blockIdx / 8 is the order within one XCD. Each XCD
    // takes super-tiles of super_m row tiles x kSuper / super_m column tiles
    // in turn, so its 32 resident workgroups share activation and weight
    // k-tiles in that XCD's L2. Row tiles enumerate (expert, tile) in expert
    // order. Fewer workgroups per activation line (8 x 4 rather than 4 x 8)
    // cut the gated GEMM's L2 hit rate from 72% to 62% but also its L1 -> L2
    // latency from 508 to 438 cycles, and it ran 6% faster.
    const int xcd = blockIdx.x & (kXcds - 1);
    const int slot = blockIdx.x / kXcds;
    const int st = (slot / kSuper) * kXcds + xcd;     // super-tile
    const int idx = slot % kSuper;
    const int sm = st % a.sm;
    const int mt = sm * a.super_m + idx % a.super_m;
    const int nt = (st / a.sm) * (kSuper / a.super_m) + idx / a.super_m;
    if (tid < 64) {
        int run = 0;
        for (int e0 = 0; e0 < a.E; e0 += 64) {
            const int e = e0 + lane;
            int v = 0;
            if (e < a.E) v = max(a.offsets[e + 1] - a.offsets[e], 0);
            v = (v + kBM - 1) / kBM;
            int x = v;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int y = __shfl_up(x, d);
                if (lane >= d) x += y;
            }
            if (e < a.E) s_tile0[e] = run + x - v;
            run += __shfl(x, 63);
        }
        if (lane == 0) s_tile0[a.E] = run;
    }
    __syncthreads();
    if (mt >= s_tile0[a.E] || nt >= a.n_tiles) return;
    int lo = 0, hi = a.E;  // s_tile0[lo] <= mt < s_tile0[hi]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (s_tile0[mid] <= mt) lo = mid; else hi = mid;
    }
    const int e = lo;
    const int row0 = a.offsets[e] + (mt - s_tile0[e]) * kBM;
    const int row_end = min(a.offsets[e + 1], a.m_total);  // rows past m_total are never touched
    if (row0 < 0 || row0 >= row_end) return;
    const int col0 = nt * tile_cols<GATED>();

    // LDS: kAStages buffers of the activation tile [kBM][kBK], then kWStages
    // of the weight tile [kBW][kBK]. A row's 16-byte chunk c lives at chunk slot
    // c ^ ((row / 2) % 8) of the row, so the 16 rows an MFMA operand read
    // serves at once fall in 16 different bank groups (rows are 128 bytes:
    // row parity picks the half of the 64 banks, the slot the group).
    const size_t K = static_cast<size_t>(a.k);
    const f16* wbase = a.w + (static_cast<size_t>(e) * a.n + col0) * K;
    const f16* w2base = GATED ? a.w2 + (static_cast<size_t>(e) * a.n + col0) * K : nullptr;
    auto cslot = [](int r, int c) { return r * kRowChunks + (c ^ ((r >> 1) & (kRowChunks - 1))); };

    // Stage loader: memory straight into LDS (buffer_load_dwordx4 ... lds).
    // Load j of wave wv fills chunk slots (j * 8 + wv) * 64 + lane of each
    // tile; the lane fetches the (row, chunk) that belongs there, so the 8
    // lanes of a row fetch its whole 128-byte line. Measured on config 8:
    // buffer loads (a 32-bit lane offset, the stage's k offset in a scalar)
    // ran the loop 7% faster than global_load_lds with 64-bit lane addresses
    // (10% with the LDS addresses in scalars),
    // and whole-line requests 8% faster than the half-line requests of 32-wide
    // k stages with three stages in flight. Rows past the expert repeat its
    // last row. Gated: weight rows 0..127 of the tile are gate rows, 128..255
    // up rows. The stage after the last reloads the last one into the buffer
    // nobody reads again.
    const int nk = a.k / kBK;
    // Buffer resources over the workgroup's rows of each operand (gated: the
    // gate rows and the up rows), so a lane's offset is 32 bits; the k
    // offset of a stage goes in the scalar offset.
    const unsigned row_bytes = static_cast<unsigned>(K) * 2u;
    const int wrows = GATED ? kBW / 2 : kBW;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<f16*>(a.a + static_cast<size_t>(row0) * K), 0, kBM * row_bytes, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<f16*>(wbase), 0, wrows * row_bytes, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rw2 = GATED ? __builtin_amdgcn_make_buffer_rsrc(
        const_cast<f16*>(w2base), 0, wrows * row_bytes, kRsrcWord3) : rw;
    // Per-lane byte offsets of load j (the k offset moves per stage).
    unsigned aoff[kLoads], woff[kLoads];
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int sl = (j * (kThreads / 64) + wv) * 64 + lane;
        const int r = sl / kRowChunks;
        const int c = (sl % kRowChunks) ^ ((r >> 1) & (kRowChunks - 1));
        const int row = min(row0 + r, row_end - 1) - row0;
        aoff[j] = static_cast<unsigned>(row) * row_bytes + 16u * c;
        woff[j] = static_cast<unsigned>(r % wrows) * row_bytes + 16u * c;
    }
    // Load j of stage ks_idx, activation (w = false) or weight tile. Gated,
    // loads j < kLoads / 2 fill the gate rows and the others the up rows.
    auto issue_load = [&](int ks_idx, int j, bool w) {
        const unsigned soff = static_cast<unsigned>(min(ks_idx, nk - 1)) * kBK * 2u;
        const int first = (j * (kThreads / 64) + wv) * 64;  // chunk slot of lane 0
        if (w) {
            f16* lx = lds + static_cast<size_t>(kAStages + ks_idx % kWStages) * kTileHalfs;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                (GATED && j >= kLoads / 2) ? rw2 : rw, to_lds(lx + first * 8),
                16, woff[j], soff, 0, 0);
        } else {
            f16* lx = lds + static_cast<size_t>(ks_idx % kAStages) * kTileHalfs;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, to_lds(lx + first * 8), 16,
                aoff[j], soff, 0, 0);
        }
    };
    // Stage s + 1 of the activation tile, then stage s + 2 of the weight tile.
    auto issue_stage = [&](int ka, int kw) {
#pragma unroll
        for (int j = 0; j < kLoads; ++j) issue_load(ka, j, false);
#pragma unroll
        for (int j = 0; j < kLoads; ++j) issue_load(kw, j, true);
    };
    // Waits until this thread's loads of the stage about to be multiplied
    // landed and its LDS reads are done, then a bare barrier. Loads are
    // issued a stage at a time, the activation tile's (stage s + 1) before the
    // weight tile's (stage s + 2), so when stage s is due the only loads of
    // this thread that may still be in flight are the kLoads weight loads of
    // stage s + 1. The empty asm statements keep the compiler from moving LDS
    // reads across the barrier.
    auto stage_ready = [&]() {
        constexpr int vm = kLoads;
        __builtin_amdgcn_s_waitcnt((0x7 << 4) | (vm & 0xF) | ((vm >> 4) << 14));  // lgkmcnt(0)
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    // Wave (wm, wn): activation rows wm*128 .. +128 as 4 MFMA column tiles
    // (j) and two 32-row weight tiles (i) at LDS weight row wrow(i):
    // plain: wn*64 + 32 i (output columns wn*64 + 32 i ..);
    // gated: i = 0 gate rows wn*32 .., i = 1 the matching up rows.
    const int wm = wv & 1, wn = wv >> 1;
    auto wrow = [&](int i) { return GATED ? i * (kBW / 2) + wn * 32 : wn * 64 + i * 32; };
    f16x acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f16x{};

    // Prologue: activation stage 0, weight stages 0 and 1 (in that order:
    // the activation loads first, as stage_ready counts).
#pragma unroll
    for (int j = 0; j < kLoads; ++j) issue_load(0, j, false);
#pragma unroll
    for (int j = 0; j < kLoads; ++j) issue_load(0, j, true);
#pragma unroll
    for (int j = 0; j < kLoads; ++j) issue_load(1, j, true);
    const int lr = lane & 31;          // MFMA row / column within a 32 tile
    const int lc = lane >> 5;          // which 8 of the 16 k of an MFMA step
    for (int kt = 0; kt < nk; ++kt) {
        // Stage kt landed in every wave's share; every wave is done with
        // stage kt - 1, whose buffers then take activation stage kt + 1 and
        // weight stage kt + 2, which load while stage kt is multiplied.
        stage_ready();
        issue_stage(kt + 1, kt + 2);
        const f16* bx = lds + static_cast<size_t>(kt % kAStages) * kTileHalfs;
        const f16* bw = lds + static_cast<size_t>(kAStages + kt % kWStages) * kTileHalfs;
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks) {
            const int c = 2 * ks + lc;
            h8 xo[4], wo[2];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = wm * 128 + j * 32 + lr;
                xo[j] = *reinterpret_cast<const h8*>(bx + cslot(r, c) * 8);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = wrow(i) + lr;
                wo[i] = *reinterpret_cast<const h8*>(bw + cslot(r, c) * 8);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma32(wo[i], xo[j], acc[i][j]);
        }
    }
    // No load may still be writing this workgroup's LDS when it exits.
    __builtin_amdgcn_s_waitcnt(0);

    // Epilogue: lane holds output row (tile j) lr and, per weight tile i,
    // columns q*8 + (lane/32)*4 + 0..3, q = 0..3.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = row0 + wm * 128 + j * 32 + lr;
        if (row >= row_end) continue;
        f16* crow = a.c + static_cast<size_t>(row) * a.n + col0;
#pragma unroll
        for (int i = 0; i < (GATED ? 1 : 2); ++i) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                h4 v;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float x = acc[i][j][q * 4 + r];
                    if (GATED) {
                        const float u = acc[1][j][q * 4 + r];
                        x = x / (1.0f + __builtin_amdgcn_exp2f(-x * kLog2e)) * u;
                    }
                    v[r] = static_cast<f16>(x);
                }
                const int col = (GATED ? wn * 32 : wn * 64 + i * 32) + q * 8 + (lane >> 5) * 4;
                *reinterpret_cast<h4*>(crow + col) = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Combine: one wave per token, 8 halfs per lane per step.
// ---------------------------------------------------------------------------
struct CombineArgs {
    const f16* y;        // [T*K][hidden]
    const float* wts;    // [T][K]
    const int* inverse;  // [T][K]
    f16* out;            // [T][hidden]
    int T;
    int K;
    int hidden;
    int rows;            // rows of y (bound on inverse)
};

__global__ __launch_bounds__(256) void moe_combine_kernel(const CombineArgs a) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.T) return;
    const int nv = a.hidden / 8;
    for (int i = lane; i < nv; i += 64) {
        float acc[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) acc[r] = 0.0f;
        for (int k = 0; k < a.K; ++k) {
            const int row = a.inverse[static_cast<size_t>(t) * a.K + k];
            if (row < 0 || row >= a.rows) continue;
            const float w = a.wts[static_cast<size_t>(t) * a.K + k];
            const h8 v = *reinterpret_cast<const h8*>(a.y + static_cast<size_t>(row) * a.hidden + 8 * i);
#pragma unroll
            for (int r = 0; r < 8; ++r) acc[r] = __builtin_fmaf(w, static_cast<float>(v[r]), acc[r]);
        }
        h8 o;
#pragma unroll
        for (int r = 0; r < 8; ++r) o[r] = static_cast<f16>(acc[r]);
        *reinterpret_cast<h8*>(a.out + static_cast<size_t>(t) * a.hidden + 8 * i) = o;
    }
}

}  // namespace
}  // namespace swiftllm

using namespace swiftllm;

extern "C" {

int swiftllm_hip_moe_expert_gemm(const void* a, const void* w, const void* w2,
                                 const int32_t* expert_offsets, int num_experts, int m_total,
                                 int n, int k, void* c, hipStream_t stream) {
    const char* who = "swiftllm_hip_moe_expert_gemm";
    if (num_experts <= 0 || m_total < 0 || n <= 0 || k <= 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: num_experts=%d m_total=%d n=%d k=%d", who,
                    num_experts, m_total, n, k);
    }
    const int cols = (w2 != nullptr) ? tile_cols<true>() : tile_cols<false>();
    // The kernel addresses a workgroup's 256 rows of each operand through a
    // buffer resource with 32-bit byte offsets: 256 * 2 * k must stay below 2^31.
    if (num_experts > kMaxE || n % cols != 0 || k % kKMult != 0 || k > kMaxK) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED,
                    "%s: num_experts=%d n=%d k=%d (supported: E <= 256, n a multiple of %d, "
                    "k a multiple of 64 up to %d)",
                    who, num_experts, n, k, cols, kMaxK);
    }
    if (!w || !expert_offsets || (m_total > 0 && (!a || !c))) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null pointer", who);
    }
    if (!aligned(a, 16) || !aligned(w, 16) || !aligned(w2, 16) || !aligned(c, 8) ||
        !aligned(expert_offsets, 4)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: misaligned pointer", who);
    }
    int rc = require_device();
    if (rc != SWIFTLLM_OK) return rc;
    if (m_total == 0) return ok();
    GemmArgs g{};
    g.a = static_cast<const f16*>(a);
    g.w = static_cast<const f16*>(w);
    g.w2 = static_cast<const f16*>(w2);
    g.offsets = expert_offsets;
    g.c = static_cast<f16*>(c);
    g.E = num_experts;
    g.m_total = m_total;
    g.n = n;
    g.k = k;
    g.m_tiles_max = (m_total + kBM - 1) / kBM + num_experts;
    g.n_tiles = n / cols;
    g.super_m = (w2 != nullptr) ? kSuperMGated : kSuperMPlain;
    const int super_n = kSuper / g.super_m;
    g.sm = (g.m_tiles_max + g.super_m - 1) / g.super_m;
    const long long supers = static_cast<long long>(g.sm) * ((g.n_tiles + super_n - 1) / super_n);
    // whole rounds of 8 super-tiles, one per XCD
    const long long grid = (supers + kXcds - 1) / kXcds * kXcds * kSuper;
    if (grid > 0x7fffffffLL) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED, "%s: %lld tiles", who, grid);
    }
    // Dynamic LDS: the activation and weight buffers (160 KiB), above the
    // default limit, so the limit is raised.
    const bool gated = (w2 != nullptr);
    const size_t lds = kLdsHalfs * sizeof(f16);
    const void* fn = gated ? reinterpret_cast<const void*>(moe_expert_gemm_kernel<true>)
                           : reinterpret_cast<const void*>(moe_expert_gemm_kernel<false>);
    hipError_t err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         static_cast<int>(lds));
    if (err != hipSuccess) return launched(err, who);
    err = gated ? launch(moe_expert_gemm_kernel<true>, dim3(static_cast<unsigned>(grid)),
                         dim3(kThreads), lds, stream, g)
                : launch(moe_expert_gemm_kernel<false>, dim3(static_cast<unsigned>(grid)),
                         dim3(kThreads), lds, stream, g);
    return launched(err, who);
}

int swiftllm_hip_moe_combine(const void* y, const float* weights, const int32_t* inverse,
                             int num_tokens, int top_k, int hidden, int y_rows, void* out,
                             hipStream_t stream) {
    const char* who = "swiftllm_hip_moe_combine";
    if (num_tokens < 0 || top_k <= 0 || hidden <= 0 || y_rows < 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: num_tokens=%d top_k=%d hidden=%d y_rows=%d",
                    who, num_tokens, top_k, hidden, y_rows);
    }
    if (hidden % 8 != 0) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED, "%s: hidden=%d (a multiple of 8 is supported)", who,
                    hidden);
    }
    if (num_tokens > 0 && (!y || !weights || !inverse || !out)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null pointer", who);
    }
    if (!aligned(y, 16) || !aligned(out, 16) || !aligned(weights, 4) || !aligned(inverse, 4)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: misaligned pointer", who);
    }
    int rc = require_device();
    if (rc != SWIFTLLM_OK) return rc;
    if (num_tokens == 0) return ok();
    CombineArgs g{static_cast<const f16*>(y), weights, inverse, static_cast<f16*>(out), num_tokens,
                  top_k, hidden, y_rows};
    return launched(launch(moe_combine_kernel, dim3((num_tokens + 3) / 4), dim3(256), 0, stream, g),
                    who);
}

}  // extern "C"
