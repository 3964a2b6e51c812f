// skv_append.hip -- KV append: scatter new tokens' K/V rows into the paged
// pools through the block tables.
//
// Replaces the reference's per-token pair of device-to-device cudaMemcpy calls
// (src/models/transformer_block.cpp:484-509), whose destination is
//     ((physical_block * block_size + slot) * num_kv_heads) * head_dim
// with physical_block = table[position / block_size], slot = position % block_size
// (src/models/transformer_block.cpp:484-499; CPU twin src/layers/attention.cpp:245-259).
// One launch moves every new token of every sequence: 16 bytes per lane,
// consecutive lanes on consecutive bytes of a row, so a row is written with
// full-width coalesced stores.  bf16 input is copied bit for bit; fp32 input is
// narrowed with the reference's round-to-nearest-even rule.
#include "skv_append.h"

#include <algorithm>

namespace skv {

// Resolve work item (sequence b, token j) to its source row and destination
// element offset; returns false when the token does not exist or its block is
// outside the table or the pool (nothing is written then).
__device__ __forceinline__ bool resolve_row(const AppendParams& p, int b, int j,
                                            int64_t& src_row, int64_t& dst_row) {
    if (p.offsets != nullptr) {
        const int first = p.offsets[b];
        if (j >= p.offsets[b + 1] - first) return false;
        src_row = static_cast<int64_t>(first) + j;
    } else {
        src_row = static_cast<int64_t>(b) * p.tokens_per_seq + j;
    }
    const int pos = (p.positions != nullptr ? p.positions[b] + p.position_bias : p.single_position) + j;
    if (pos < 0) return false;
    const int blk = pos / p.block_size;
    if (blk >= p.max_blocks) return false;
    const int64_t pb = p.tables[static_cast<int64_t>(b) * p.max_blocks + blk];
    if (pb < 0 || pb >= p.total_blocks) return false;
    dst_row = pb * p.block_size + (pos % p.block_size);
    return true;
}

// Vector path: rows are a multiple of 8 elements, every lane moves 8 elements.
template <bool FP32_SRC>
__global__ __launch_bounds__(256) void kv_append_vec_kernel(AppendParams p) {
    const int chunks = p.row_elems >> 3;
    const int64_t items = static_cast<int64_t>(p.num_seqs) * p.tokens_per_seq * chunks;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t it = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; it < items;
         it += stride) {
        const int64_t t = it / chunks;
        const int ch = static_cast<int>(it - t * chunks);
        const int b = static_cast<int>(t / p.tokens_per_seq);
        const int j = static_cast<int>(t - static_cast<int64_t>(b) * p.tokens_per_seq);
        int64_t src_row, dst_row;
        if (!resolve_row(p, b, j, src_row, dst_row)) continue;
        const int64_t src = src_row * p.row_elems + (ch << 3);
        const int64_t dst = dst_row * p.row_elems + (ch << 3);
        uint4 kw, vw;
        if constexpr (FP32_SRC) {
            const float4* ks = reinterpret_cast<const float4*>(static_cast<const float*>(p.k_new) + src);
            const float4* vs = reinterpret_cast<const float4*>(static_cast<const float*>(p.v_new) + src);
            const float4 k0 = ks[0], k1 = ks[1], v0 = vs[0], v1 = vs[1];
            kw = make_uint4(pack_bf16x2(k0.x, k0.y), pack_bf16x2(k0.z, k0.w),
                            pack_bf16x2(k1.x, k1.y), pack_bf16x2(k1.z, k1.w));
            vw = make_uint4(pack_bf16x2(v0.x, v0.y), pack_bf16x2(v0.z, v0.w),
                            pack_bf16x2(v1.x, v1.y), pack_bf16x2(v1.z, v1.w));
        } else {
            kw = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.k_new) + src);
            vw = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.v_new) + src);
        }
        *reinterpret_cast<uint4*>(p.k_pool + dst) = kw;
        *reinterpret_cast<uint4*>(p.v_pool + dst) = vw;
    }
}

// Scalar path for rows that are not a multiple of 8 elements or unaligned inputs.
template <bool FP32_SRC>
__global__ __launch_bounds__(256) void kv_append_scalar_kernel(AppendParams p) {
    const int64_t items = static_cast<int64_t>(p.num_seqs) * p.tokens_per_seq * p.row_elems;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t it = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; it < items;
         it += stride) {
        const int64_t t = it / p.row_elems;
        const int e = static_cast<int>(it - t * p.row_elems);
        const int b = static_cast<int>(t / p.tokens_per_seq);
        const int j = static_cast<int>(t - static_cast<int64_t>(b) * p.tokens_per_seq);
        int64_t src_row, dst_row;
        if (!resolve_row(p, b, j, src_row, dst_row)) continue;
        const int64_t src = src_row * p.row_elems + e;
        const int64_t dst = dst_row * p.row_elems + e;
        if constexpr (FP32_SRC) {
            p.k_pool[dst] = static_cast<uint16_t>(f32_to_bf16_bits(static_cast<const float*>(p.k_new)[src]));
            p.v_pool[dst] = static_cast<uint16_t>(f32_to_bf16_bits(static_cast<const float*>(p.v_new)[src]));
        } else {
            p.k_pool[dst] = static_cast<const uint16_t*>(p.k_new)[src];
            p.v_pool[dst] = static_cast<const uint16_t*>(p.v_new)[src];
        }
    }
}

}  // namespace skv

using namespace skv;

extern "C" int skv_kv_append(const void* k_new, const void* v_new, int src_dtype,
                             uint16_t* k_pool, uint16_t* v_pool, int64_t total_blocks,
                             const int32_t* block_tables, int max_blocks_per_seq,
                             const int32_t* positions, const int32_t* token_offsets,
                             int num_seqs, int tokens_per_seq, int num_kv_heads, int head_dim,
                             int block_size, void* stream) {
    SKV_REQUIRE(num_seqs >= 0 && tokens_per_seq >= 0,
                "skv_kv_append: negative sequence or token count");
    if (num_seqs == 0 || tokens_per_seq == 0) return SKV_OK;
    SKV_REQUIRE(k_new && v_new && k_pool && v_pool && block_tables && positions,
                "skv_kv_append: NULL pointer");
    SKV_REQUIRE(src_dtype == SKV_DTYPE_BF16 || src_dtype == SKV_DTYPE_FP32,
                "skv_kv_append: unknown source dtype %d", src_dtype);
    SKV_REQUIRE(total_blocks > 0 && max_blocks_per_seq > 0 && num_kv_heads > 0 && head_dim > 0 &&
                    block_size > 0,
                "skv_kv_append: dimensions must be positive");
    const int64_t row = static_cast<int64_t>(num_kv_heads) * head_dim;
    SKV_REQUIRE(row <= (1 << 24), "skv_kv_append: row of %lld elements is too large",
                static_cast<long long>(row));

    AppendParams p{k_new, v_new, k_pool, v_pool, total_blocks, block_tables, max_blocks_per_seq,
                   positions, 0, 0, token_offsets, num_seqs, tokens_per_seq, static_cast<int>(row),
                   block_size};
    return launch_append(p, src_dtype, static_cast<hipStream_t>(stream));
}

extern "C" int skv_kv_append_token(const void* k_row, const void* v_row, int src_dtype,
                                   uint16_t* k_pool, uint16_t* v_pool, int64_t total_blocks,
                                   const int32_t* block_table, int table_len, int position,
                                   int num_kv_heads, int head_dim, int block_size, void* stream) {
    SKV_REQUIRE(k_row && v_row && k_pool && v_pool && block_table,
                "skv_kv_append_token: NULL pointer");
    SKV_REQUIRE(src_dtype == SKV_DTYPE_BF16 || src_dtype == SKV_DTYPE_FP32,
                "skv_kv_append_token: unknown source dtype %d", src_dtype);
    SKV_REQUIRE(total_blocks > 0 && table_len > 0 && num_kv_heads > 0 && head_dim > 0 &&
                    block_size > 0 && position >= 0,
                "skv_kv_append_token: invalid dimensions or position");
    SKV_REQUIRE(position / block_size < table_len,
                "skv_kv_append_token: no KV page for position %d", position);
    const int64_t row = static_cast<int64_t>(num_kv_heads) * head_dim;
    SKV_REQUIRE(row <= (1 << 24), "skv_kv_append_token: row too large");
    AppendParams p{k_row, v_row, k_pool, v_pool, total_blocks, block_table, table_len, nullptr, 0,
                   position, nullptr, 1, 1, static_cast<int>(row), block_size};
    return launch_append(p, src_dtype, static_cast<hipStream_t>(stream));
}

namespace skv {
int launch_append(const AppendParams& p, int src_dtype, hipStream_t s) {
    const int64_t row = p.row_elems;
    const int num_seqs = p.num_seqs, tokens_per_seq = p.tokens_per_seq;
    const void* k_new = p.k_new;
    const void* v_new = p.v_new;
    const uint16_t* k_pool = p.k_pool;
    const uint16_t* v_pool = p.v_pool;
    const bool vec = (row % 8) == 0 && aligned16(k_new) && aligned16(v_new) &&
                     aligned16(k_pool) && aligned16(v_pool);
    const int64_t items = static_cast<int64_t>(num_seqs) * tokens_per_seq * (vec ? row / 8 : row);
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(cdiv<int64_t>(items, 256), 8192));
    if (vec) {
        if (src_dtype == SKV_DTYPE_FP32)
            kv_append_vec_kernel<true><<<grid, 256, 0, s>>>(p);
        else
            kv_append_vec_kernel<false><<<grid, 256, 0, s>>>(p);
    } else {
        if (src_dtype == SKV_DTYPE_FP32)
            kv_append_scalar_kernel<true><<<grid, 256, 0, s>>>(p);
        else
            kv_append_scalar_kernel<false><<<grid, 256, 0, s>>>(p);
    }
    return check_launch("kv_append_kernel");
}
}  // namespace skv
