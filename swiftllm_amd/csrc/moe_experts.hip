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
//   columns; gated: 128 gate rows and their 128 up rows), k in stages of 64
//   (one 128-byte line of each row) copied from memory straight into LDS by
//   buffer loads (two activation and three weight buffers, 160 KiB; rows
//   swizzled by 16-byte chunk so the operand reads are free of bank
//   conflicts); eight waves of 128 x 64 in two ping-pong groups (one
//   multiplies while the other loads), each on v_mfma_f32_32x32x16_f16 with
//   the weight as the MFMA's row operand, so a lane ends with 4 consecutive
//   output columns of one row (8-byte stores) and, gated, holds the gate
//   and up value of each of its columns. The 256 x 256 tile does 128 FLOP per byte staged, so L2 feeds
//   the matrix cores at ~20 TB/s. Tiles are (expert, 256-row tile, column
//   tile); a workgroup finds its expert from the offsets, and the grid is
//   sized for the worst case (rows / 256 whole tiles plus min(E, rows / 129)
//   tails of more than 128 rows); surplus workgroups exit at once. An
//   expert's last rows past its whole tiles, when at most 128, go to a second,
//   HBM-bound kernel instead (thin tiles, below): a decode batch gives every
//   expert only such rows.
// combine: out[t, :] = sum_k weights[t, k] * y[inverse[t, k], :] in fp32
//   (k ascending, fused multiply-add), rounded once to fp16; entries with
//   inverse outside [0, rows of y) contribute nothing. One wave per token;
//   for top-k <= 8 (except 5 and 7) a kernel with k fixed at compile time
//   issues all of a lane's row loads for several chunks before adding.

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
constexpr int kAStages = 2;     // LDS buffers of the activation tile
constexpr int kWStages = 3;     // LDS buffers of the weight tile (its lines miss L2 more)
constexpr int kThreads = 512;   // 8 waves: 2 (rows) x 4 (weight rows), 128 x 64 each
constexpr int kRowChunks = kBK / 8;                        // 16-byte chunks per tile row
// Cache policy of a buffer load: the nt bit (streaming), for the thin
// kernel's weight rows, which it reads once per call.
constexpr int kNontemporal = 2;
constexpr int kTileChunks = kBM * kRowChunks;              // chunks per operand tile
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
// with its experts' short tails in the thin kernel, each expert has 4 row
// tiles, and the gate and up GEMM runs 2% faster per call at 4 x 8 (a
// super-tile's rows are one expert's) than at 8 x 4; before, when the short
// tails were further row tiles, 8 x 4 (or 16 x 2) had been 4% faster than
// 4 x 8. The down GEMM varies by about 1% over all shapes, fastest at 16 x 2.
// Shapes of more than 32 workgroups (16 x 4, 12 x 4) ran 10% slower.
constexpr int kSuperMGated = 4;
constexpr int kSuperMPlain = 16;
constexpr int kSuper = 32;

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

__device__ __forceinline__ f16x mfma32(h8 a, h8 b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Output columns per workgroup tile: 256 plain, 128 gated (each column needs
// its gate and its up row).
template <bool GATED>
constexpr int tile_cols() { return GATED ? kBW / 2 : kBW; }

// An expert's rows past its last whole 256-row tile form its tail. A tail of
// at most kThinRows rows goes to the thin kernel below instead of a 256-row
// tile: such a tile costs a whole tile's matrix work and weight staging for a
// few rows (config 8: 4 of 36 row tiles hold 5 to 31 rows), and a batch of
// decode tokens gives every expert only such a tail (a 512-token batch, top-2
// of 8 experts: about 128 rows each).
constexpr int kThinRows = 128;

// Row tiles of an expert with `count` rows in the main kernel.
__device__ __forceinline__ int main_row_tiles(int count) {
    const int tail = count % kBM;
    return count / kBM + (tail > kThinRows ? 1 : 0);
}

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
    // order.
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
            if (e < a.E) v = main_row_tiles(max(a.offsets[e + 1] - a.offsets[e], 0));
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

    // Ping-pong. The 8 waves form two groups, waves 0-3 and 4-7; waves w
    // and w + 4 share a SIMD. Each group alternates a memory phase (its
    // operand fragments of one k stage from LDS into registers, and its
    // share of the stage loads) with a compute phase (the stage's 32 MFMAs
    // on those registers), and the groups run one phase apart, every phase
    // closed by a workgroup barrier: while one wave of a SIMD multiplies,
    // the other loads, so the matrix pipe is fed from alternating waves
    // instead of both waves stalling on their reads together. Group 0 loads
    // the activation tiles, group 1 the weight tiles, each in its memory
    // phase. Measured on config 8's gated / down GEMM (one box): 1993 /
    // 1184 us with both groups in step (each stage behind one barrier),
    // 1812 / 1059 us ping-pong; the same loop without any global loads ran
    // 1508 / 854 us, so what is left is the loads' issue, not their waits.
    //
    // Stage loads go from memory straight into LDS (buffer_load_dwordx4 ...
    // lds): load j of a group's wave gw fills chunk slots (j * 4 + gw) * 64
    // + lane of the tile; the lane fetches the (row, chunk) that belongs
    // there, so the 8 lanes of a row fetch its whole 128-byte line. Rows past
    // the expert repeat its last row. Gated: weight rows 0..127 of the tile
    // are gate rows, 128..255 up rows (loads j < 4 and j >= 4). Measured
    // before: buffer loads (a 32-bit lane offset, the stage's k offset in a
    // scalar) ran the loop 7% faster than global_load_lds with 64-bit lane
    // addresses, and whole-line requests 8% faster than the half-line
    // requests of 32-wide k stages.
    //
    // Phases are counted by barriers. Group 0's memory phase of stage s ends
    // at barrier 2 + 2s and its compute phase at 3 + 2s; group 1 runs one
    // barrier later (its memory phase of stage s ends at 3 + 2s). Buffers:
    //   activation stage s in A buffer s % 2, loaded by group 0 in its
    //     memory phase of s - 1 (the buffer's previous stage, s - 2, was read
    //     by group 0 and group 1 before barrier 2s - 1) and waited for
    //     (vmcnt(0)) at the end of its compute phase of s - 1, before
    //     barrier 2s + 1, a phase before group 0 reads it;
    //   weight stage s in W buffer s % 3, loaded by group 1 in its memory
    //     phase of s - 2 (stage s - 3's readers are done by barrier 2s - 3)
    //     and waited for at the end of its memory phase of s - 1 (vmcnt(8):
    //     the 8 loads of stage s + 1, issued after them, may still fly), before
    //     barrier 2s + 1.
    // Every wave passes 2 + 2 nk barriers: group 1 one extra at the start,
    // group 0 one at the end.
    constexpr int kGroupLoads = kTileChunks / (kThreads / 2);  // loads per thread per tile
    const int nk = a.k / kBK;
    const int grp = wv >> 2;
    const int gw = wv & 3;  // wave within its group
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
    // Per-lane byte offsets of load j within the group's tile (the k offset
    // moves per stage).
    unsigned off[kGroupLoads];
#pragma unroll
    for (int j = 0; j < kGroupLoads; ++j) {
        const int sl = (j * 4 + gw) * 64 + lane;
        const int r = sl / kRowChunks;
        const int c = (sl % kRowChunks) ^ ((r >> 1) & (kRowChunks - 1));
        const int row = grp == 0 ? min(row0 + r, row_end - 1) - row0 : r % wrows;
        off[j] = static_cast<unsigned>(row) * row_bytes + 16u * c;
    }
    // Activation stage s lives in LDS buffer s % kAStages, weight stage s in
    // buffer kAStages + s % kWStages. (The addresses are spelled out at each
    // use: a lambda returning a pointer into the extern __shared__ array,
    // called from the other lambdas, made hipcc's host pass drop the
    // kernel's launch stub without a diagnostic.)
    // All of the group's loads of stage s (group 0: activations, 1: weights).
    auto issue_stage = [&](int s) {
        const unsigned soff = static_cast<unsigned>(s) * kBK * 2u;
#pragma unroll
        for (int j = 0; j < kGroupLoads; ++j) {
            const int first = (j * 4 + gw) * 64;  // chunk slot of lane 0
            if (grp == 0) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, to_lds(lds + static_cast<size_t>(s % kAStages) * kTileHalfs + first * 8), 16, off[j],
                                                         soff, 0, 0);
            } else {
                __builtin_amdgcn_raw_ptr_buffer_load_lds((GATED && j >= kGroupLoads / 2) ? rw2 : rw,
                                                         to_lds(lds + static_cast<size_t>(kAStages + s % kWStages) * kTileHalfs + first * 8), 16, off[j],
                                                         soff, 0, 0);
            }
        }
    };
    // A bare barrier; the empty asm statements keep the compiler from moving
    // memory operations across it, the scheduling barriers anything else.
    auto barrier = [] {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };
    constexpr int kWaitAll = 0;                  // vmcnt(0) expcnt(0) lgkmcnt(0)
    constexpr int kWaitLds = 0xc07f;             // lgkmcnt(0) only
    constexpr int kWaitLdsVm8 = 0x0078;          // lgkmcnt(0) vmcnt(8)
    static_assert(kGroupLoads == 8, "kWaitLdsVm8 leaves one stage's loads in flight");

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
    const int lr = lane & 31;          // MFMA row / column within a 32 tile
    const int lc = lane >> 5;          // which 8 of the 16 k of an MFMA step
    h8 xo[kBK / 16][4], wo[kBK / 16][2];  // one stage's fragments: [k step][tile]
    auto read_stage = [&](int s) {
        const f16* bx = lds + static_cast<size_t>(s % kAStages) * kTileHalfs;
        const f16* bw = lds + static_cast<size_t>(kAStages + s % kWStages) * kTileHalfs;
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks) {
            const int c = 2 * ks + lc;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                xo[ks][j] = *reinterpret_cast<const h8*>(bx + cslot(wm * 128 + j * 32 + lr, c) * 8);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                wo[ks][i] = *reinterpret_cast<const h8*>(bw + cslot(wrow(i) + lr, c) * 8);
            }
        }
    };

    // Prologue: stage 0 of both tiles, then group 1 starts weight stage 1
    // and takes its extra barrier.
    issue_stage(0);
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    barrier();
    if (grp == 1) {
        if (nk > 1) issue_stage(1);
        barrier();
    }
    for (int kt = 0; kt < nk; ++kt) {
        // Memory phase.
        read_stage(kt);
        if (grp == 0) {
            if (kt + 1 < nk) issue_stage(kt + 1);
            __builtin_amdgcn_s_waitcnt(kWaitLds);
        } else if (kt + 2 < nk) {
            issue_stage(kt + 2);
            __builtin_amdgcn_s_waitcnt(kWaitLdsVm8);  // weight stage kt + 1 landed
        } else {
            __builtin_amdgcn_s_waitcnt(kWaitAll);
        }
        barrier();
        // Compute phase.
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma32(wo[ks][i], xo[ks][j], acc[i][j]);
        if (grp == 0) __builtin_amdgcn_s_waitcnt(kWaitAll);  // activation stage kt + 1 landed
        barrier();
    }
    if (grp == 0) barrier();
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
// Thin tiles: the tail of at most kThinRows rows of each expert, times
// thin_out output columns per workgroup. A tail this short makes the tile a
// stream of its weight rows (HBM-bound, 2 * tail FLOP per weight byte), so the
// kernel is built for bytes in flight: a ring of thin_stages 64-k stages in
// LDS, each the tile's weight rows and the tail's rows (padded to 128 by
// repeating the last one), loaded by buffer loads straight into LDS in whole
// 128-byte lines with the main kernel's chunk swizzle, thin_stages - 1 of
// them in flight. The four waves read their operands from the stage and run
// v_mfma_f32_32x32x16_f16 with 32 weight rows as the row operand and 32 tail
// rows as the column operand, as in the main kernel, so a lane ends with 4
// consecutive output columns of one row per tail tile. The padding rows cost
// MFMA work and L2 hits only: the kernel is bound by streaming the weights. Gated: the stage's
// first thin_out weight rows are gate rows, the next thin_out the matching up
// rows; a wave multiplies both for its columns and forms the SiLU product in
// the epilogue.
// ---------------------------------------------------------------------------
constexpr int kThinThreads = 256;   // 4 waves
constexpr int kThinLds = 160 * 1024;

// Output columns per workgroup: 128 plain (4 waves of 32 columns), 64 gated
// (2 column tiles of 32, each for two waves that share its tail tiles), so
// that the gated GEMM's n / 64 x E workgroups of a decode batch (1792 for
// Mixtral's 14336 x 8) fill whole rounds on 256 CUs.
template <bool GATED>
constexpr int thin_out() { return GATED ? 64 : 128; }

// A thin tile's shape for a tail of at most 32 NTT rows (NTT = 1, 2 or 4
// tiles of 32): a stage holds the tile's TW weight rows and 32 NTT tail rows
// (the last one repeated), and as many stages as fit in the LDS make the
// ring (8 for NTT = 1, 6 for 2, 5 for 4), so short tails, which load fewer
// rows per stage, keep more stages in flight.
template <bool GATED, int NTT>
struct Thin {
    static constexpr int OUT = thin_out<GATED>();
    static constexpr int TW = GATED ? 2 * OUT : OUT;              // weight rows per stage
    static constexpr int ROWS = TW + 32 * NTT;                     // stage rows
    static constexpr int L = ROWS * kRowChunks / kThinThreads;    // loads per thread per stage
    static constexpr size_t SH = static_cast<size_t>(ROWS) * kBK; // stage size in halves
    static constexpr int NS = kThinLds / static_cast<int>(SH * sizeof(f16));
    static constexpr int CT = OUT / 32;                           // column tiles
    static constexpr int NT = (NTT * CT + 3) / 4;                 // tail tiles per wave
    static_assert(ROWS * kRowChunks % kThinThreads == 0 && (TW * kRowChunks) % 64 == 0 &&
                      (OUT * kRowChunks) % 64 == 0,
                  "each load instruction stays inside one operand");
    static_assert(NS >= 3 && (NS - 2) * L < 64, "ring and vmcnt field");
};

// Stage ks of a thin tile into LDS buffer buf: load j of wave wv fills chunk
// slots j * 256 + wv * 64 + lane (8 rows: tile weight rows, then tail rows).
// A __device__ function rather than a lambda: a lambda issuing these buffer
// loads made hipcc's host pass drop the kernel's launch stub.
template <bool GATED, int NTT>
__device__ __forceinline__ void thin_issue(f16* lds, __amdgpu_buffer_rsrc_t rx, __amdgpu_buffer_rsrc_t rw,
                                           __amdgpu_buffer_rsrc_t rw2, const unsigned* off, int wv,
                                           int ks, int buf) {
    using C = Thin<GATED, NTT>;
    static_assert((C::TW * kRowChunks) % kThinThreads == 0 && (C::OUT * kRowChunks) % kThinThreads == 0,
                  "the rows of load j lie in one operand for every wave");
    const unsigned soff = static_cast<unsigned>(ks) * kBK * 2u;
#pragma unroll
    for (int j = 0; j < C::L; ++j) {
        // Load j of every wave reads rows of one operand (rj: its first row
        // for wave 0), so the choice below is made at compile time. The
        // weight rows are read once per call and go nontemporal; the tail
        // rows, which every column tile of the expert reads, stay cached.
        const int rj = j * kThinThreads / kRowChunks;
        f16* dst = lds + static_cast<size_t>(buf) * C::SH + (j * kThinThreads + wv * 64) * 8;
        if (rj >= C::TW) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, to_lds(dst), 16, off[j], soff, 0, 0);
        } else {
            __builtin_amdgcn_raw_ptr_buffer_load_lds((GATED && rj >= C::OUT) ? rw2 : rw, to_lds(dst), 16,
                                                     off[j], soff, 0, kNontemporal);
        }
    }
}

// One thin tile: expert e's tail rows [row0, row_end) (tail = their count)
// times output columns [col0, col0 + OUT).
template <bool GATED, int NTT>
__device__ __forceinline__ void thin_tile(const GemmArgs& a, f16* lds, int e, int row0, int row_end,
                                          int tail, int col0, int wv, int lane) {
    using C = Thin<GATED, NTT>;
    constexpr int NW = GATED ? 2 : 1;            // weight row tiles per wave
    constexpr int NT = C::NT;
    const int ct = wv % C::CT;                   // this wave's column tile
    const int t0 = (wv / C::CT) * NT;            // and its first tail tile
    const size_t K = static_cast<size_t>(a.k);
    const unsigned row_bytes = static_cast<unsigned>(K) * 2u;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<f16*>(a.a + static_cast<size_t>(row0) * K), 0, 32 * NTT * row_bytes, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<f16*>(a.w + (static_cast<size_t>(e) * a.n + col0) * K), 0, C::OUT * row_bytes,
        kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rw2 = GATED ? __builtin_amdgcn_make_buffer_rsrc(
        const_cast<f16*>(a.w2 + (static_cast<size_t>(e) * a.n + col0) * K), 0, C::OUT * row_bytes,
        kRsrcWord3) : rw;
    // Byte offset of load j of this lane: stage row r = slot / 8 (weight
    // rows, then the tail rows), the 8 lanes of a row its 128-byte line.
    unsigned off[C::L];
#pragma unroll
    for (int j = 0; j < C::L; ++j) {
        const int sl = j * kThinThreads + wv * 64 + lane;
        const int r = sl / kRowChunks;
        const int c = (sl % kRowChunks) ^ ((r >> 1) & (kRowChunks - 1));
        const int orow = r < C::TW ? r % C::OUT : min(row0 + (r - C::TW), row_end - 1) - row0;
        off[j] = static_cast<unsigned>(orow) * row_bytes + 16u * c;
    }
    const int lr = lane & 31;
    const int lc = lane >> 5;
    f16x acc[NW][NT];
#pragma unroll
    for (int i = 0; i < NW; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[i][t] = f16x{};

    const int nk = a.k / kBK;
    constexpr int NS = C::NS;
    // With a one-tile tail, workgroups start their k walk at different
    // stages (and wrap), so that at any moment they read different k offsets
    // of their rows: the weight rows of a stage sit k * 2 bytes apart (8 KiB
    // for k = 4096), and the same offset in every row would load the same
    // HBM channels. Step kt reads stage (kt + rot) % nk; the sum is the same
    // set of stages. Longer tails keep an expert's workgroups in step, since
    // they then share its many tail rows in L2. Measured (one box): 64-token
    // decode batch 497 -> 489 us per call with the rotation; rotating every
    // shape made a 512-token batch's down GEMM 208 -> 260 us.
    const int rot = NTT == 1 ? static_cast<int>((blockIdx.x * 37u + blockIdx.y * 11u) %
                                                static_cast<unsigned>(nk))
                             : 0;
    auto stage = [&](int kt) { const int s = kt + rot; return s >= nk ? s - nk : s; };
    // Stages 0 .. NS - 2 in flight; steps past the last reload the last one
    // (in bounds, never read as a stage), so every step issues one stage.
#pragma unroll
    for (int s = 0; s < NS - 1; ++s)
        thin_issue<GATED, NTT>(lds, rx, rw, rw2, off, wv, stage(min(s, nk - 1)), s);
    for (int kt = 0; kt < nk; ++kt) {
        wait_vm<(NS - 2) * C::L>();   // this wave's loads of stage kt landed
        // Everyone's, and everyone is done with stage kt - 1. The empty asm
        // statements keep the compiler from moving memory operations across.
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        thin_issue<GATED, NTT>(lds, rx, rw, rw2, off, wv, stage(min(kt + NS - 1, nk - 1)),
                               (kt + NS - 1) % NS);   // into step kt - 1's buffer
        const f16* st = lds + static_cast<size_t>(kt % NS) * C::SH;
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks) {
            const int c = 2 * ks + lc;
            h8 xf[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int r = C::TW + 32 * min(t0 + t, NTT - 1) + lr;
                xf[t] = *reinterpret_cast<const h8*>(st + (r * kRowChunks + (c ^ ((r >> 1) & (kRowChunks - 1)))) * 8);
            }
#pragma unroll
            for (int i = 0; i < NW; ++i) {
                const int r = i * C::OUT + ct * 32 + lr;
                const h8 wf = *reinterpret_cast<const h8*>(st + (r * kRowChunks + (c ^ ((r >> 1) & (kRowChunks - 1)))) * 8);
                // Every tile unconditionally: a branch per MFMA made the
                // allocator copy the accumulators between AGPRs and VGPRs
                // around each one (2x slower gated). Padding rows repeat the
                // last tail row, so their results are finite and not stored.
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[i][t] = mfma32(wf, xf[t], acc[i][t]);
            }
        }
    }
    // No load may still be writing this workgroup's LDS when it exits.
    __builtin_amdgcn_s_waitcnt(0);

    // Lane holds tail rows 32 (t0 + t) + lr and output columns col0 + ct*32 + q*8 + lc*4 + 0..3.
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int row = row0 + 32 * (t0 + t) + lr;
        if (t0 + t >= NTT || row >= row_end) continue;
        f16* crow = a.c + static_cast<size_t>(row) * a.n + col0 + ct * 32;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            h4 v;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float x = acc[0][t][q * 4 + r];
                if constexpr (GATED) {
                    const float u = acc[1][t][q * 4 + r];
                    x = x / (1.0f + __builtin_amdgcn_exp2f(-x * kLog2e)) * u;
                }
                v[r] = static_cast<f16>(x);
            }
            *reinterpret_cast<h4*>(crow + q * 8 + lc * 4) = v;
        }
    }
}

template <bool GATED>
__global__ __launch_bounds__(kThinThreads) void moe_expert_thin_kernel(const GemmArgs a) {
    extern __shared__ __align__(16) f16 lds[];
    const int e = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int count = max(a.offsets[e + 1] - a.offsets[e], 0);
    const int tail = count % kBM;
    if (tail == 0 || tail > kThinRows) return;
    const int row0 = a.offsets[e] + (count - tail);
    const int row_end = min(a.offsets[e + 1], a.m_total);
    if (row0 < 0 || row0 >= row_end) return;
    const int col0 = blockIdx.x * thin_out<GATED>();   // the grid covers n / OUT column tiles
    // Uniform over the workgroup: the tile shape for this tail.
    if (tail <= 32) thin_tile<GATED, 1>(a, lds, e, row0, row_end, tail, col0, wv, lane);
    else if (tail <= 64) thin_tile<GATED, 2>(a, lds, e, row0, row_end, tail, col0, wv, lane);
    else thin_tile<GATED, 4>(a, lds, e, row0, row_end, tail, col0, wv, lane);
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

// Top-k known at compile time (KC = K <= 8). The bound is bytes in flight, so
// each lane issues the loads of U row chunks of all KC rows before the first
// multiply-add: 16·U·KC bytes per lane. Each row of y is read exactly once per
// call, so the loads are nontemporal. A row index outside [0, rows) gives no
// term: its load reads row 0 (rows > 0 on this path), and the term becomes
// 0 · (−0) = −0, which leaves every accumulator bit for bit as it was, so
// the loads need no branches. Terms add in k order in fp32, then
// one fp16 rounding, as in the generic kernel below.
template <int KC>
__global__ __launch_bounds__(256) void moe_combine_kernel_k(const CombineArgs a) {
    constexpr int U = KC <= 2 ? 4 : (KC <= 4 ? 2 : 1);
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.T) return;
    const int nv = a.hidden / 8;
    const h8* src[KC];
    float w[KC];
    bool use[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k) {
        const int row = a.inverse[static_cast<size_t>(t) * KC + k];
        use[k] = row >= 0 && row < a.rows;
        w[k] = use[k] ? a.wts[static_cast<size_t>(t) * KC + k] : 0.0f;
        src[k] = reinterpret_cast<const h8*>(a.y + static_cast<size_t>(use[k] ? row : 0) * a.hidden);
    }
    h8* dst = reinterpret_cast<h8*>(a.out + static_cast<size_t>(t) * a.hidden);
    for (int i0 = lane; i0 < nv; i0 += 64 * U) {
        h8 v[U][KC];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = min(i0 + 64 * u, nv - 1);
#pragma unroll
            for (int k = 0; k < KC; ++k) v[u][k] = __builtin_nontemporal_load(src[k] + i);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (i0 + 64 * u >= nv) break;
            float acc[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) acc[r] = 0.0f;
#pragma unroll
            for (int k = 0; k < KC; ++k) {
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    acc[r] = __builtin_fmaf(w[k], use[k] ? static_cast<float>(v[u][k][r]) : -0.0f,
                                            acc[r]);
                }
            }
            h8 o;
#pragma unroll
            for (int r = 0; r < 8; ++r) o[r] = static_cast<f16>(acc[r]);
            dst[i0 + 64 * u] = o;
        }
    }
}

// Any top-k: one row load in flight per lane.
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
    // Row tiles of the main grid: whole 256-row tiles hold 256 rows each and
    // a tail left there holds more than kThinRows, so at most m / 256 of the
    // first and min(E, m / (kThinRows + 1)) of the second (expert offsets
    // partition the m_total rows).
    g.m_tiles_max = m_total / kBM + std::min(num_experts, m_total / (kThinRows + 1));
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
    if (grid > 0) {  // none when every expert's rows fit one thin tail (m_total <= 128)
        err = gated ? launch(moe_expert_gemm_kernel<true>, dim3(static_cast<unsigned>(grid)),
                             dim3(kThreads), lds, stream, g)
                    : launch(moe_expert_gemm_kernel<false>, dim3(static_cast<unsigned>(grid)),
                             dim3(kThreads), lds, stream, g);
        if (err != hipSuccess) return launched(err, who);
    }
    // The experts' short tails (at most kThinRows rows), which the main grid
    // leaves out; workgroups of experts without one exit at once.
    const dim3 thin(static_cast<unsigned>(n / (gated ? thin_out<true>() : thin_out<false>())),
                    static_cast<unsigned>(num_experts));
    const size_t tl = kThinLds;
    const void* tf = gated ? reinterpret_cast<const void*>(moe_expert_thin_kernel<true>)
                           : reinterpret_cast<const void*>(moe_expert_thin_kernel<false>);
    err = hipFuncSetAttribute(tf, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(tl));
    if (err != hipSuccess) return launched(err, who);
    err = gated ? launch(moe_expert_thin_kernel<true>, thin, dim3(kThinThreads), tl, stream, g)
                : launch(moe_expert_thin_kernel<false>, thin, dim3(kThinThreads), tl, stream, g);
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
    const dim3 grid((num_tokens + 3) / 4);
    hipError_t e;
    switch (y_rows > 0 ? top_k : 0) {
        case 1: e = launch(moe_combine_kernel_k<1>, grid, dim3(256), 0, stream, g); break;
        case 2: e = launch(moe_combine_kernel_k<2>, grid, dim3(256), 0, stream, g); break;
        case 3: e = launch(moe_combine_kernel_k<3>, grid, dim3(256), 0, stream, g); break;
        case 4: e = launch(moe_combine_kernel_k<4>, grid, dim3(256), 0, stream, g); break;
        case 6: e = launch(moe_combine_kernel_k<6>, grid, dim3(256), 0, stream, g); break;
        case 8: e = launch(moe_combine_kernel_k<8>, grid, dim3(256), 0, stream, g); break;
        default: e = launch(moe_combine_kernel, grid, dim3(256), 0, stream, g); break;
    }
    return launched(e, who);
}

}  // extern "C"
