// skv_append.h -- internal: parameters of the KV append kernels, shared by the
// append entry points and the decode entry point that appends before decoding.
#pragma once

#include "skv_common.h"

namespace skv {

struct AppendParams {
    const void* k_new;
    const void* v_new;
    uint16_t* k_pool;
    uint16_t* v_pool;
    int64_t total_blocks;
    const int32_t* tables;
    int max_blocks;
    const int32_t* positions; // [num_seqs] (+ position_bias), or nullptr -> single_position
    int position_bias;
    int single_position;
    const int32_t* offsets;   // [num_seqs + 1] or nullptr
    int num_seqs;
    int tokens_per_seq;       // tokens per sequence (upper bound when offsets != nullptr)
    int row_elems;            // num_kv_heads * head_dim
    int block_size;
};

// Launches the vector (16 B per lane) or scalar append kernel on stream s.
int launch_append(const AppendParams& p, int src_dtype, hipStream_t s);

}  // namespace skv
