// Status plumbing and host-only entry points of libswiftllm_hip.so.
//
// The status codes mirror CudaError (crates/swiftllm-cuda/src/lib.rs:16-42);
// the message stands for the String payload those variants carry.

#include <cstdarg>
#include <cstdio>
#include <string>

#include "common.hpp"

namespace swiftllm {
namespace {
thread_local int t_status = SWIFTLLM_OK;
thread_local std::string t_message;
}  // namespace

int ok() {
    t_status = SWIFTLLM_OK;
    t_message.clear();
    return SWIFTLLM_OK;
}

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    t_status = code;
    t_message = buf;
    return code;
}

int require_device() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        return fail(SWIFTLLM_ERR_DEVICE_NOT_FOUND, "HIP device not found");
    }
    return SWIFTLLM_OK;
}

int launched(hipError_t err, const char* what) {
    if (err != hipSuccess) {
        return fail(SWIFTLLM_ERR_KERNEL, "%s: launch failed: %s", what,
                    hipGetErrorString(err));
    }
    return ok();
}

}  // namespace swiftllm

using namespace swiftllm;

extern "C" {

int swiftllm_hip_last_error(void) { return t_status; }

const char* swiftllm_hip_last_error_message(void) { return t_message.c_str(); }

const char* swiftllm_hip_version(void) { return "0.1.0 gfx950"; }

int swiftllm_hip_device_check(void) {
    int rc = require_device();
    return rc == SWIFTLLM_OK ? ok() : rc;
}

// kv_cache.rs:186-216. Positions are usize on the host; the ABI narrows the
// resulting slots to int32 (bindings.rs:100) and refuses what does not fit.
int swiftllm_hip_slot_mapping(const uint64_t* block_table, size_t table_len,
                              size_t block_size, size_t start_pos,
                              size_t num_tokens, int32_t* out) {
    if (block_size == 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "block_size must be > 0");
    }
    if (num_tokens > 0 && (out == nullptr || block_table == nullptr)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "null pointer");
    }
    for (size_t i = 0; i < num_tokens; ++i) {
        const size_t pos = start_pos + i;
        const size_t block_idx = pos / block_size;
        const size_t block_offset = pos % block_size;
        if (block_idx >= table_len) {
            return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                        "Block %zu not allocated for sequence", block_idx);
        }
        const uint64_t physical = block_table[block_idx];
        const unsigned __int128 slot =
            static_cast<unsigned __int128>(physical) * block_size + block_offset;
        if (slot > static_cast<unsigned __int128>(INT32_MAX)) {
            return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                        "slot of position %zu does not fit in int32", pos);
        }
        out[i] = static_cast<int32_t>(slot);
    }
    return ok();
}

// Flattens BatchedCacheMetadata.block_tables / context_lens
// (kv_cache.rs:250-286) into the int32 arrays the decode kernels read.
int swiftllm_hip_pack_block_tables(const uint64_t* block_ids,
                                   const uint64_t* table_offsets,
                                   const uint64_t* context_lens,
                                   size_t num_seqs, size_t block_size,
                                   size_t max_blocks_per_seq,
                                   int32_t* block_tables_out,
                                   int32_t* context_lens_out) {
    if (block_size == 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "block_size must be > 0");
    }
    if (num_seqs == 0) return ok();
    if (!table_offsets || !context_lens || !block_tables_out ||
        !context_lens_out) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "null pointer");
    }
    if (max_blocks_per_seq > static_cast<size_t>(INT32_MAX)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                    "max_blocks_per_seq does not fit in int32");
    }
    // block_ids may be null only when every table is empty.
    if (!block_ids && table_offsets[num_seqs] != table_offsets[0]) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "null block_ids");
    }
    for (size_t s = 0; s < num_seqs; ++s) {
        const uint64_t begin = table_offsets[s];
        const uint64_t end = table_offsets[s + 1];
        if (end < begin) {
            return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                        "table_offsets not ascending at sequence %zu", s);
        }
        const uint64_t len = end - begin;
        const uint64_t ctx = context_lens[s];
        const uint64_t need = (ctx + block_size - 1) / block_size;
        if (len > max_blocks_per_seq || need > max_blocks_per_seq) {
            return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                        "sequence %zu needs %llu blocks > max_blocks_per_seq %zu",
                        s, static_cast<unsigned long long>(len > need ? len : need),
                        max_blocks_per_seq);
        }
        if (need > len) {
            return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                        "sequence %zu: context %llu needs %llu blocks, table has %llu",
                        s, static_cast<unsigned long long>(ctx),
                        static_cast<unsigned long long>(need),
                        static_cast<unsigned long long>(len));
        }
        if (ctx > static_cast<uint64_t>(INT32_MAX)) {
            return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                        "context length of sequence %zu does not fit in int32", s);
        }
        int32_t* row = block_tables_out + s * max_blocks_per_seq;
        for (uint64_t j = 0; j < len; ++j) {
            const uint64_t id = block_ids[begin + j];
            if (id > static_cast<uint64_t>(INT32_MAX)) {
                return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                            "block id %llu does not fit in int32",
                            static_cast<unsigned long long>(id));
            }
            row[j] = static_cast<int32_t>(id);
        }
        for (uint64_t j = len; j < max_blocks_per_seq; ++j) row[j] = 0;
        context_lens_out[s] = static_cast<int32_t>(ctx);
    }
    return ok();
}

}  // extern "C"
