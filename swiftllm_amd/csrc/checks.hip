// Check entry point for the wave-level reductions the kernels are built on,
// so that they can be held lane by lane against a sequential reference: the
// reference's butterflies (paged_attention.cu:17-31, 32 lanes, mask
// 0xffffffff) become, on 64-lane waves,
//   max_over_kg / sum_over_kg (attention_core.hpp): lanes l, l ^ 16, l ^ 32,
//       l ^ 48 on the permlane16/32 swaps (the softmax row max and sum of
//       the MFMA accumulator layout, decode and prefill);
//   wave_max / wave_sum (common.hpp): all 64 lanes by xor shuffles (the
//       split-K reduce);
//   wave_inclusive_scan (common.hpp): the 64-lane prefix sum (MoE dispatch,
//       split-K item lists).
// The functions run here are the ones the kernels inline, not copies.

#include "attention_core.hpp"

namespace swiftllm {
namespace {

struct ReduceCheckArgs {
    const float* x;
    const int* xi;
    float* out;  // [n][4][64]: max_over_kg, sum_over_kg, wave_max, wave_sum
    int* scan;   // [n][64]
    int n;
};

__global__ __launch_bounds__(256) void wave_reduce_check_kernel(const ReduceCheckArgs a) {
    const int row = blockIdx.x * 4 + static_cast<int>(threadIdx.x >> 6);
    if (row >= a.n) return;  // whole waves
    const int lane = threadIdx.x & 63;
    const float v = a.x[static_cast<size_t>(row) * 64 + lane];
    float* o = a.out + static_cast<size_t>(row) * 256;
    o[lane] = attn::max_over_kg(v);
    o[64 + lane] = attn::sum_over_kg(v);
    o[128 + lane] = wave_max(v);
    o[192 + lane] = wave_sum(v);
    a.scan[static_cast<size_t>(row) * 64 + lane] =
        wave_inclusive_scan(a.xi[static_cast<size_t>(row) * 64 + lane], lane);
}

}  // namespace
}  // namespace swiftllm

using namespace swiftllm;

extern "C" {

int swiftllm_hip_wave_reduce_check(const float* x, const int32_t* xi, int num_rows, float* out,
                                   int32_t* scan, hipStream_t stream) {
    const char* who = "swiftllm_hip_wave_reduce_check";
    if (num_rows < 0) return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: num_rows=%d", who, num_rows);
    if (num_rows > 0 && (!x || !xi || !out || !scan)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null pointer", who);
    }
    if (!aligned(x, 4) || !aligned(xi, 4) || !aligned(out, 4) || !aligned(scan, 4)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: misaligned pointer", who);
    }
    int rc = require_device();
    if (rc != SWIFTLLM_OK) return rc;
    if (num_rows == 0) return ok();
    ReduceCheckArgs a{x, xi, out, scan, num_rows};
    return launched(launch(wave_reduce_check_kernel, dim3((num_rows + 3) / 4), dim3(256), 0, stream, a),
                    who);
}

}  // extern "C"
