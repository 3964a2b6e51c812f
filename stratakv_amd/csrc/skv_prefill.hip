// skv_prefill.hip -- chunked prefill attention over the paged KV cache: a
// chunk of new tokens per sequence, already appended to the pools, each token
// attending causally to every earlier position of its sequence (its own chunk
// included).
//
// Semantics: src/layers/attention.cpp:197-337 (PagedAttention::forward with
// more than one new token: token i of the chunk sits at position
// p = context - chunk + i and attends to positions 0..p through the page
// table).  The reference computes it on the CPU only.
//
// Kernel (block_size 16, head_dim 64/128, G = Hq/Hkv in {1, 2, 4, 8, 16}):
// * A workgroup of 8 wavefronts owns 256 query rows = the G heads of one kv
//   head for 256/G consecutive tokens of one sequence (row r = token * G +
//   head); wavefront w owns rows 32w..32w+31 as two 16-row column groups.
//   Every K/V byte staged in LDS serves all 256 rows.
// * Keys are walked 64 at a time (four 16-token blocks) up to the tile's last
//   position, through two LDS buffers, one barrier per step.  While the
//   current step is computed, the next step's K rows go straight from memory
//   into the other buffer (buffer_load_dwordx4 ... lds: no registers, no LDS
//   store instruction) and its V rows into registers, converted to fp16 and
//   stored after the compute.  K rows are unpadded, each 16-byte chunk c of
//   row r stored at chunk position c ^ (r % chunks per row) (the DMA writes
//   lane i's 16 bytes at position i, so lane i loads the chunk that belongs
//   there); V rows are padded by 32 bytes.  Both make the operand reads below
//   conflict-free (a 16-byte padding of K had left half of the K reads' LDS
//   cycles in bank conflicts).  The heaviest tiles (the latest tokens of each
//   sequence) are scheduled first.
// * The step loop keeps its K/V loads in flight through the compute: they are
//   unconditional buffer loads through a per-(wavefront, block) descriptor that
//   spans exactly the block's existing rows (rows past the context and absent
//   blocks read as zeros without a memory access), the block ids come from
//   table entries held 64 per VGPR and read with v_readlane (no scalar load,
//   whose out-of-order return would turn every LDS wait into lgkmcnt(0)), and
//   the query operands are complete before the loop.  With per-lane branches
//   around the loads and a scalar table read per block, the compiler had
//   waited for all of them (vmcnt(0)) before the step's first MFMA.
// * Little scalar work per step: the CU's 8 wavefronts share one scalar unit
//   and all reach the step's load issue together after the barrier.  Each
//   wavefront stages half of one block per step; its byte offset and extent
//   come precomputed from the table window (once per 64 entries, on the
//   VALU), and a step carries a 4-bit mask of its existing blocks instead of
//   a 64-bit mask of keys.  (Four block ids, their products and a key mask
//   per wavefront and step had taken ~19 % of the step.)
// * S^T = K Q^T on the matrix cores (v_mfma_f32_16x16x32_bf16: keys as rows,
//   query rows as columns), so each lane holds the scores of ONE query row:
//   the causal/validity mask, the row max (2 shuffles) and the rescale of that
//   row's output are lane-local.  Each K operand read serves both column
//   groups.  An fp32 query is split into hi + lo bf16 parts (two MFMAs), so
//   its products keep ~16 significant bits.
// * O^T += V^T P^T, also on the matrix cores: P goes from the S^T output
//   registers straight into the B operand (keys {4j..4j+3, 16+4j..16+4j+3} of
//   lane group j), and the V^T operand comes out of the row-major V tile with
//   the LDS transpose read (ds_read_b64_tr_b16: in each 16-lane group, lane
//   4a + c receives element c of the 8-byte rows addressed by lanes a, a+4,
//   a+8, a+12), in the same key order.  This product runs in fp16
//   (v_mfma_f32_16x16x32_f16, fp32 accumulation): V is converted from bf16
//   as it is staged (exact for |v| in [2^-14, 65504]; below, an absolute error
//   under 2^-25), P is rounded to the nearest fp16 (11 significant bits,
//   against bf16's 8).  A tile that stages a V element above 65504 (finite
//   in bf16, or infinite) has its rows recomputed in fp32 instead.
// * Online softmax in the exp2 domain with lazy rescaling (threshold 2^8, so
//   P <= 256 stays well inside the fp16 range).
// Other shapes run a simple kernel (one wavefront per token and query head).
#include "skv_common.h"

#include <algorithm>
#include <cmath>

namespace skv {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct PrefillParams {
    const void* q;             // [N][Hq][HD] bf16 or fp32
    const uint16_t* k;
    const uint16_t* v;
    int64_t total_blocks;
    const int32_t* tables;     // [B][max_blocks]
    int max_blocks;
    const int32_t* offsets;    // [B + 1] query rows of each sequence's chunk
    const int32_t* lens;       // [B] context length including the chunk
    int B, Hq, Hkv, HD, bs;
    float qscale;              // softmax scale * log2(e)
    float* out;                // [N][Hq][HD] fp32
    int tile_tokens;           // tokens per workgroup tile (MFMA kernel)
};

constexpr int kPrefillMaxBatch = 4096;
constexpr float kPrefillLazy = 8.0f;

__device__ __forceinline__ int chunk_tokens(const PrefillParams& p, int b) {
    return max(0, p.offsets[b + 1] - p.offsets[b]);
}

// Tiles of tile_tokens tokens per sequence, prefix-summed into T_s[0..B] by
// wavefront 0 (the same scan for every workgroup), T_s[B + 1] = the largest
// per-sequence count; returns the total.
__device__ int prefill_tile_scan(const PrefillParams& p, int* T_s) {
    const int lane = threadIdx.x;
    if (lane < 64) {
        int carry = 0, most = 0;
        for (int b0 = 0; b0 < p.B; b0 += 64) {
            const int b = b0 + lane;
            int v = b < p.B ? cdiv(chunk_tokens(p, b), p.tile_tokens) : 0;
            int mx = v;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) mx = max(mx, __shfl_xor(mx, o, 64));
            most = max(most, mx);
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int u = __shfl_up(v, o, 64);
                if (lane >= o) v += u;
            }
            if (b < p.B) T_s[b + 1] = carry + v;
            carry += __shfl(v, 63, 64);
        }
        if (lane == 0) {
            T_s[0] = 0;
            T_s[p.B + 1] = most;
        }
    }
    __syncthreads();
    return T_s[p.B];
}

__device__ __forceinline__ int find_tile_seq(const int* T, int B, int tile) {
    int lo = 0, hi = B;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (T[mid] <= tile) lo = mid; else hi = mid;
    }
    return lo;
}

// ---------------------------------------------------------------------------
// MFMA kernel.  Lane layouts (16x16x32 MFMA): lane (t, j) = (lane % 16,
// lane / 16).  A operand of S^T: key row t (+16 kt), head-dim chunk 4cc + j;
// B operand: query row t of column group c, chunk 4cc + j; S^T output: keys
// 4j + i (+16 kt), query row t.  P^T B operand: query row t, keys {4j..4j+3,
// 16+4j..16+4j+3} of a 32-key chunk; V^T A operand: dim 16 dt + t, the same 8
// keys; O^T output: dims 16 dt + 4j + i, query row t.
// ---------------------------------------------------------------------------
constexpr int kPrefillWaves = 8;
constexpr int kPrefillRows = kPrefillWaves * 32;   // query rows per workgroup
constexpr int kPrefillKeys = 64;                   // keys per step

template <int HD>
struct PrefillLds {
    // K rows unpadded: 16-byte chunk c of row r stored at chunk position
    // c ^ (r % chunks per row).
    static constexpr int KRS = HD * 2;             // K row stride (bytes)
    static constexpr int VRS = HD * 2 + 32;        // V row stride (bytes)
    static constexpr int KB = kPrefillKeys * KRS;
    static constexpr int BUF = KB + kPrefillKeys * VRS;
    static constexpr int TOTAL = 2 * BUF;          // two buffers; the tile scan follows
    __device__ static constexpr int k_chunk(int row, int c) {
        return row * KRS + (c ^ (row & (HD / 8 - 1))) * 16;
    }
};

// 16 bytes per lane from a buffer straight into LDS (buffer_load_dwordx4 ...
// lds): lane i writes bytes [16 i, 16 i + 16) after `lds_base` (wave-uniform).
// The host pass of the compiler has no form of this builtin, so its call sits
// in the device pass only.
// s_waitcnt operand for vmcnt(0) alone (gfx9 encoding: expcnt 7 and lgkmcnt 15
// are their "don't wait" values): the wave's LDS DMA has landed.
constexpr int kWaitVmcnt0 = 0x0F70;

__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rsrc, unsigned char* lds_base, int voffset) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds_base, 16, voffset, 0,
                                             0, 0);
#endif
}

typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
    const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

// fp32 recomputation of wavefront wv's rows of a tile (the MFMA kernel's
// path when a V element of the tile is beyond the fp16 range): lanes over 64
// keys for the scores, over head dims for P.V, the keys' probabilities and
// rows broadcast by shuffles.  Row r = token r / G, head r % G of kv head kvh.
template <int HD, int G, bool QF32>
__device__ __forceinline__ void prefill_rows_fp32(const PrefillParams& p, int b, int kvh, int wv, int ntok, int tok0,
                                               int base_pos, int keys_end, const int32_t* table) {
    const int lane = threadIdx.x & 63;
    const int64_t row_elems = static_cast<int64_t>(p.Hkv) * HD;
    for (int rr = 0; rr < 32; ++rr) {
        const int r = wv * 32 + rr;
        const int qtok = r / G;
        if (qtok >= ntok) break;
        const int64_t qoff = (static_cast<int64_t>(p.offsets[b] + tok0 + qtok) * p.Hq + kvh * G + r % G) * HD;
        const int nkeys = min(base_pos + qtok + 1, keys_end);
        float m = -INFINITY, l = 0.0f;
        float acc[HD / 64];
#pragma unroll
        for (int k = 0; k < HD / 64; ++k) acc[k] = 0.0f;
        for (int t0 = 0; t0 < nkeys; t0 += 64) {
            const int tk = t0 + lane;
            float score = -INFINITY;
            int64_t roff = -1;
            if (tk < nkeys) {
                const int64_t pb = table[tk >> 4];
                if (pb >= 0 && pb < p.total_blocks) {
                    roff = (pb * 16 + (tk & 15)) * row_elems + static_cast<int64_t>(kvh) * HD;
                    float dot = 0.0f;
                    for (int d = 0; d < HD; ++d) {
                        const float qv = QF32 ? static_cast<const float*>(p.q)[qoff + d]
                                              : bf16_to_f32(static_cast<const uint16_t*>(p.q)[qoff + d]);
                        dot = fmaf(qv, bf16_to_f32(p.k[roff + d]), dot);
                    }
                    score = dot * p.qscale;
                }
            }
            const float mn = fmaxf(m, wave_max(score));
            const float ms = mn == -INFINITY ? 0.0f : mn;
            const float alpha = fast_exp2(m - ms);
            const float pp = fast_exp2(score - ms);
            l = l * alpha + wave_sum(pp);
            m = mn;
#pragma unroll
            for (int k = 0; k < HD / 64; ++k) acc[k] *= alpha;
            const int cnt = min(64, nkeys - t0);
            for (int jj = 0; jj < cnt; ++jj) {
                const int64_t vr = (static_cast<int64_t>(__shfl(static_cast<int>(roff >> 32), jj, 64)) << 32) |
                                   static_cast<uint32_t>(__shfl(static_cast<int>(roff), jj, 64));
                const float pj = __shfl(pp, jj, 64);
                if (vr < 0) continue;
#pragma unroll
                for (int k = 0; k < HD / 64; ++k) acc[k] = fmaf(pj, bf16_to_f32(p.v[vr + lane + 64 * k]), acc[k]);
            }
        }
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float* o = p.out + qoff;
#pragma unroll
        for (int k = 0; k < HD / 64; ++k) o[lane + 64 * k] = acc[k] * inv;
    }
}

template <int HD, int G, bool QF32>
__global__ __launch_bounds__(64 * kPrefillWaves) void prefill_mfma_kernel(PrefillParams p) {
    using Lds = PrefillLds<HD>;
    constexpr int KS = kPrefillKeys;
    static_assert(KS == 64, "one validity bit per key of a step in a 64-bit mask");
    constexpr int CH = HD / 8;              // 16-byte chunks per row
    constexpr int NKC = HD / 32;            // 32-dim steps of S
    constexpr int NDT = HD / 16;            // 16-dim tiles of O
    constexpr int QP = QF32 ? 2 : 1;
    constexpr int QT = kPrefillRows / G;    // tokens per tile
    constexpr int NT = 64 * kPrefillWaves;
    constexpr int LOADS = KS * CH / NT;     // 16-byte chunks per thread per step (K, and V)
    static_assert(LOADS >= 1 && KS * CH % NT == 0, "load split");

    extern __shared__ __align__(16) unsigned char lds[];
    int* T_s = reinterpret_cast<int*>(lds + Lds::TOTAL);   // [B + 3]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t = lane & 15, j = lane >> 4;
    const int kvh = blockIdx.x % p.Hkv;
    const int slot = blockIdx.x / p.Hkv;

    if (tid == 0) T_s[p.B + 2] = 0;   // set when the tile's rows must be recomputed in fp32
    const int ntiles = prefill_tile_scan(p, T_s);
    if (slot >= ntiles) return;
    // Heaviest first: with equal tile counts, the last tile of every sequence,
    // then the one before, ...; otherwise the global order reversed.
    const int most = T_s[p.B + 1];
    int b, tile_in_seq;
    if (most * p.B == ntiles) {
        b = slot % p.B;
        tile_in_seq = most - 1 - slot / p.B;
    } else {
        const int tile = ntiles - 1 - slot;
        b = find_tile_seq(T_s, p.B, tile);
        tile_in_seq = tile - T_s[b];
    }
    const int n = chunk_tokens(p, b);
    const int L = p.lens[b];
    const int tok0 = tile_in_seq * QT;
    const int ntok = min(QT, n - tok0);
    const int base_pos = L - n + tok0;                 // position of the tile's first token
    const int last_pos = base_pos + ntok - 1;
    const int nb_seq = min(cdiv(max(L, 0), 16), p.max_blocks);
    const int keys_end = min(last_pos + 1, nb_seq * 16);  // keys [0, keys_end) may be read
    const int32_t* table = p.tables + static_cast<int64_t>(b) * p.max_blocks;
    const int64_t row_stride = static_cast<int64_t>(p.Hkv) * HD;
    // Position of this wave's first query row (its rows' positions only grow).
    const int wave_first_pos = base_pos + (wv * 32) / G;

    // This lane's two query rows (column t of the two column groups).
    int qpos[2];
    int64_t qrow[2];
    bool live[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int r = wv * 32 + c * 16 + t;
        const int qtok = r / G, qhead = kvh * G + r % G;
        live[c] = qtok < ntok;
        qpos[c] = live[c] ? base_pos + qtok : -1;      // -1: every key masked
        qrow[c] = static_cast<int64_t>(p.offsets[b] + tok0 + qtok) * p.Hq + qhead;
    }

    bf16x8_t qop[QP][2][NKC];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int cc = 0; cc < NKC; ++cc) {
            u32x4_t hi = {0u, 0u, 0u, 0u}, lo = {0u, 0u, 0u, 0u};
            if (live[c]) {
                const int64_t off = qrow[c] * HD + (4 * cc + j) * 8;
                if constexpr (QF32) {
                    const float4* qp = reinterpret_cast<const float4*>(static_cast<const float*>(p.q) + off);
                    const float4 a0 = qp[0], a1 = qp[1];
                    const float x[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                    uint32_t hb[4], lb[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        hb[e] = pack2_bf16(x[2 * e], x[2 * e + 1]);
                        lb[e] = pack2_bf16(x[2 * e] - __uint_as_float(hb[e] << 16),
                                           x[2 * e + 1] - __uint_as_float(hb[e] & 0xFFFF0000u));
                    }
                    hi = u32x4_t{hb[0], hb[1], hb[2], hb[3]};
                    lo = u32x4_t{lb[0], lb[1], lb[2], lb[3]};
                } else {
                    hi = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p.q) + off);
                }
            }
            qop[0][c][cc] = __builtin_bit_cast(bf16x8_t, hi);
            if constexpr (QF32) qop[QP - 1][c][cc] = __builtin_bit_cast(bf16x8_t, lo);
        }
    // The query operands are complete here (the empty asm reads them), so no
    // wait for these loads is left for the step loop to merge with its own.
#pragma unroll
    for (int qp = 0; qp < QP; ++qp)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int cc = 0; cc < NKC; ++cc) {
                const u32x4_t w = __builtin_bit_cast(u32x4_t, qop[qp][c][cc]);
                asm volatile("" ::"v"(w.x), "v"(w.y), "v"(w.z), "v"(w.w));
            }

    // Table entries 64 per VGPR (lane i holds entry tb + i), the next 64
    // loaded one chunk ahead.  Once per 64 entries each lane turns its entry
    // into the block's byte offset and the bytes of its existing rows (0 for
    // an absent block, an id outside the pool, or a block at or past
    // keys_end), and a ballot gives wmask (bit i: block tb + i exists); a step
    // then reads its block with three v_readlane and no scalar arithmetic on
    // the id.  The loop issues no scalar load (whose out-of-order return would
    // make every LDS wait a full lgkmcnt(0)) and no K/V load waits on a table
    // read.
    static_assert(kPrefillWaves * 8 == KS && LOADS * (64 / CH) == 8, "a wavefront stages half a block per step");
    const int64_t row_bytes = row_stride * 2;
    const int nb_tab = max(nb_seq, 1);
    auto tab_load = [&](int first) -> int { return table[min(first + lane, nb_tab - 1)]; };
    int tb = 0;
    int tvn = tab_load(64);
    uint32_t off_lo = 0, off_hi = 0;   // this lane's window entry: byte offset of the block's rows
    int nrec_v = 0;                    // and the bytes of its existing rows of one kv head
    uint64_t wmask = 0;
    auto set_window = [&](int e) {
        const bool ok = (tb + lane) * 16 < keys_end && e >= 0 && e < p.total_blocks;
        const uint64_t off = ok ? static_cast<uint64_t>(e) * static_cast<uint64_t>(16 * row_bytes) : 0ull;
        off_lo = static_cast<uint32_t>(off);
        off_hi = static_cast<uint32_t>(off >> 32);
        nrec_v = ok ? static_cast<int>(min(16, keys_end - (tb + lane) * 16) * row_bytes) : 0;
        wmask = __ballot(ok);
    };
    set_window(tab_load(0));
    auto window = [&](int s) {   // blocks 4 s .. 4 s + 3; steps are visited in order
        if (4 * s - tb >= 64) {
            tb += 64;
            set_window(tvn);
            tvn = tab_load(tb + 64);
        }
    };
    // Bit hb set when block hb of step s exists.
    auto step_nib = [&](int s) -> uint32_t { return static_cast<uint32_t>(wmask >> (4 * s - tb)) & 0xFu; };
    // Loads of a step: wavefront wv stages rows 8 (wv & 1) .. + 7 of the
    // step's block wv >> 1 (LOADS passes of 64 / CH rows, CH consecutive lanes
    // per row slice), through a buffer descriptor that spans exactly the
    // block's existing rows (0 for an absent block), so rows that do not exist
    // load as zeros and every load is issued unconditionally.
    const int blk_w = wv >> 1;
    const uint16_t* const kbase = p.k + static_cast<int64_t>(kvh) * HD;
    const uint16_t* const vbase = p.v + static_cast<int64_t>(kvh) * HD;
    int row_w[LOADS], voff_w[LOADS];
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
        row_w[u] = 8 * (wv & 1) + u * (64 / CH) + lane / CH;   // row within the block
        voff_w[u] = static_cast<int>(row_w[u] * row_bytes + (lane % CH) * 16);
    }
    // K goes straight into LDS buffer `buf` (buffer_load ... lds): lane i of
    // pass u writes the 16 bytes at LDS row lr0 + i / CH, chunk position
    // i % CH, so it loads the block row's chunk (i % CH) ^ (row % CH) -- the
    // swizzled layout, realised through the source addresses.
    int kvoff_w[LOADS];
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
        const int lr = 16 * blk_w + row_w[u];
        kvoff_w[u] = static_cast<int>(row_w[u] * row_bytes + (((lane % CH) ^ (lr & (CH - 1))) * 16));
    }
    auto load_step = [&](int s, int buf, u32x4_t (&vr)[LOADS]) {
        const int slot = 4 * s + blk_w - tb;
        const uint64_t off = static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(off_lo, slot))) |
                             static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(off_hi, slot))) << 32;
        const int nrec = __builtin_amdgcn_readlane(nrec_v, slot);
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<unsigned char*>(reinterpret_cast<const unsigned char*>(kbase)) + off, 0, nrec, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<unsigned char*>(reinterpret_cast<const unsigned char*>(vbase)) + off, 0, nrec, 0x00020000);
        unsigned char* kb = lds + buf * Lds::BUF;
#pragma unroll
        for (int u = 0; u < LOADS; ++u) {
            const int lr0 = 16 * blk_w + 8 * (wv & 1) + u * (64 / CH);   // first LDS row of this pass
            lds_dma16(rk, kb + lr0 * Lds::KRS, kvoff_w[u]);
        }
#pragma unroll
        for (int u = 0; u < LOADS; ++u)
            vr[u] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, voff_w[u], 0, 0));
    };
    // Rows of keys that do not exist are stored as zeros (V must not carry
    // NaN from unused slots into 0 * V).
    // V is stored as fp16 (exact for |v| in [2^-14, 65504]; smaller values
    // keep an absolute error below 2^-25); vmax tracks the largest |V| this
    // thread stored.
    float vmax = 0.0f;
    auto store_step = [&](int buf, const u32x4_t (&vr)[LOADS]) {
        unsigned char* kb = lds + buf * Lds::BUF;
        unsigned char* vb = kb + Lds::KB;
#pragma unroll
        for (int u = 0; u < LOADS; ++u) {
            const int lr = 16 * blk_w + row_w[u], lc = lane % CH;
            u32x4_t w;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float lo = __uint_as_float(vr[u][e] << 16), hi = __uint_as_float(vr[u][e] & 0xFFFF0000u);
                vmax = fmaxf(vmax, fmaxf(fabsf(lo), fabsf(hi)));
                w[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, f16x2_t));
            }
            *reinterpret_cast<u32x4_t*>(vb + lr * Lds::VRS + lc * 16) = w;
        }
    };

    f32x4_t acc[NDT][2];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[dt][c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m[2] = {-INFINITY, -INFINITY};   // reference max of each row (log2 units)
    float lsum[2] = {0.0f, 0.0f};          // this lane's share of each row's denominator

    const int nsteps = cdiv(keys_end, KS);
    u32x4_t vr[LOADS];
    uint32_t nib_cur = 0, nib_next = 0;   // blocks of the current and next step that exist
    if (nsteps > 0) {
        nib_cur = step_nib(0);
        load_step(0, 0, vr);
        store_step(0, vr);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);   // this wave's K rows are in LDS
    __syncthreads();
    for (int st = 0; st < nsteps; ++st) {
        const int cur = st & 1;
        if (st + 1 < nsteps) {   // in flight during compute
            window(st + 1);
            nib_next = step_nib(st + 1);
            load_step(st + 1, cur ^ 1, vr);
        }
        const unsigned char* kb = lds + cur * Lds::BUF;
        const unsigned char* vb = kb + Lds::KB;
        const int k0 = st * KS;

        // ---- S^T tiles: s[c][kt] = scores of keys 16 kt + 4j + i, row t of group c
        f32x4_t s[2][KS / 16];
#pragma unroll
        for (int kt = 0; kt < KS / 16; ++kt) {
            s[0][kt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            s[1][kt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int cc = 0; cc < NKC; ++cc) {
                const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(kb + Lds::k_chunk(kt * 16 + t, 4 * cc + j));
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int qp = 0; qp < QP; ++qp)
                        s[c][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qop[qp][c][cc], s[c][kt], 0, 0, 0);
            }
        }

        // ---- online softmax per row, P^T operands (fp16).
        // Scores stay unscaled: qscale > 0, so max(s) * qscale is the max of
        // the scaled scores, and the exponent is one fma.  Steps whose keys
        // all exist and precede the wave's first query position (all but the
        // diagonal steps of a tile) skip the mask.
        const bool need_mask = !(nib_cur == 0xFu && keys_end - k0 >= KS && k0 + KS - 1 <= wave_first_pos);
        f16x8_t pf[2][KS / 32];   // P^T operands
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            float sc[KS / 4];
#pragma unroll
            for (int kt = 0; kt < KS / 16; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) sc[kt * 4 + i] = s[c][kt][i];
            if (need_mask) {
                // Key kl exists when its block does (bit kt of nib_cur) and
                // k0 + kl < keys_end; it is visible when k0 + kl <= qpos.
                const int lim = min(qpos[c] - k0, keys_end - k0 - 1);
#pragma unroll
                for (int kt = 0; kt < KS / 16; ++kt) {
                    const bool present = (nib_cur >> kt) & 1u;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        sc[kt * 4 + i] = present && kt * 16 + 4 * j + i <= lim ? sc[kt * 4 + i] : -INFINITY;
                }
            }
            float mb = sc[0];
#pragma unroll
            for (int e = 1; e < KS / 4; ++e) mb = fmaxf(mb, sc[e]);
            mb = xor32_max(xor16_max(mb)) * p.qscale;
            if (mb > m[c] + kPrefillLazy) {   // lane-local: the row's state lives in this lane
                const float alpha = m[c] == -INFINITY ? 0.0f : fast_exp2(m[c] - mb);
                m[c] = mb;
                lsum[c] *= alpha;
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[dt][c][i] *= alpha;
            }
            const float ms = m[c] == -INFINITY ? 0.0f : m[c];
            float pr[KS / 4];
#pragma unroll
            for (int e = 0; e < KS / 4; ++e) {
                pr[e] = fast_exp2(fmaf(sc[e], p.qscale, -ms));
                lsum[c] += pr[e];
            }
            // 32-key chunk h: keys {4j..4j+3} = kt 2h, {16+4j..} = kt 2h+1.
#pragma unroll
            for (int h = 0; h < KS / 32; ++h) {
                uint32_t hw[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    hw[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                        f32x2_t{pr[8 * h + 2 * e], pr[8 * h + 2 * e + 1]}, f16x2_t));
                pf[c][h] = __builtin_bit_cast(f16x8_t, u32x4_t{hw[0], hw[1], hw[2], hw[3]});
            }
        }

        // ---- O^T += V^T P^T; V^T through the LDS transpose read.  Source
        // lane 16g + a + 4e addresses key 32h + 16r + 4g + e, dims 16dt + 4a.
        const int ga = lane & 3, ge = (lane >> 2) & 3, gg = lane >> 4;
#pragma unroll
        for (int h = 0; h < KS / 32; ++h) {
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                v4s_t part[2];
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const int key = 32 * h + 16 * r + 4 * gg + ge;
                    const unsigned char* src = vb + key * Lds::VRS + (16 * dt + 4 * ga) * 2;
                    part[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) v4s_t*)(src));
                }
                const u32x4_t w = {__builtin_bit_cast(uint2, part[0]).x, __builtin_bit_cast(uint2, part[0]).y,
                                   __builtin_bit_cast(uint2, part[1]).x, __builtin_bit_cast(uint2, part[1]).y};
                const f16x8_t a = __builtin_bit_cast(f16x8_t, w);
#pragma unroll
                for (int c = 0; c < 2; ++c)
                    acc[dt][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pf[c][h], acc[dt][c], 0, 0, 0);
            }
        }

        if (st + 1 < nsteps) store_step(cur ^ 1, vr);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);   // the next step's K rows are in LDS
        __syncthreads();
        nib_cur = nib_next;
    }

    // A V element beyond the fp16 range (finite above 65504, or infinite)
    // anywhere in the tile: its rows are recomputed in fp32.
    if (vmax > 65504.0f) T_s[p.B + 2] = 1;
    __syncthreads();
    if (T_s[p.B + 2] != 0) {
        prefill_rows_fp32<HD, G, QF32>(p, b, kvh, wv, ntok, tok0, base_pos, keys_end, table);
        return;
    }

    // ---- output: O[row][dims 16 dt + 4j + i] = acc / l
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const float ltot = xor32_sum(xor16_sum(lsum[c]));
        if (live[c]) {
            const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
            float* o = p.out + qrow[c] * HD;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
                *reinterpret_cast<float4*>(o + dt * 16 + 4 * j) =
                    make_float4(acc[dt][c][0] * inv, acc[dt][c][1] * inv, acc[dt][c][2] * inv, acc[dt][c][3] * inv);
        }
    }
}

// ---------------------------------------------------------------------------
// Generic kernel: one wavefront per (query token, query head); keys 64 at a
// time (lanes over keys for the scores, over head dims for P.V), online
// softmax.  Any block size, head_dim <= 512.
// ---------------------------------------------------------------------------
template <bool QF32>
__global__ __launch_bounds__(64) void prefill_generic_kernel(PrefillParams p, int num_tokens) {
    constexpr int DPL = 512 / 64;
    __shared__ float q_s[512];
    __shared__ float p_s[64];
    __shared__ int64_t row_s[64];
    const int lane = threadIdx.x;
    const int h = blockIdx.x % p.Hq;
    const int tokg = blockIdx.x / p.Hq;
    if (tokg >= num_tokens) return;
    // Sequence of the token: offsets[b] <= tokg < offsets[b + 1].
    int lo = 0, hi = p.B;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (p.offsets[mid] <= tokg) lo = mid; else hi = mid;
    }
    const int b = lo;
    const int n = chunk_tokens(p, b);
    const int pos = p.lens[b] - n + (tokg - p.offsets[b]);
    const int HD = p.HD, bs = p.bs;
    const int kvh = h / (p.Hq / p.Hkv);
    const int64_t row_elems = static_cast<int64_t>(p.Hkv) * HD;
    const int32_t* table = p.tables + static_cast<int64_t>(b) * p.max_blocks;
    const int64_t qoff = (static_cast<int64_t>(tokg) * p.Hq + h) * HD;
    for (int d = lane; d < HD; d += 64) {
        const float qv = QF32 ? static_cast<const float*>(p.q)[qoff + d]
                              : bf16_to_f32(static_cast<const uint16_t*>(p.q)[qoff + d]);
        q_s[d] = qv * p.qscale;
    }
    __syncthreads();
    float m = -INFINITY, l = 0.0f;
    float acc[DPL];
#pragma unroll
    for (int k = 0; k < DPL; ++k) acc[k] = 0.0f;
    const int nkeys = min(pos + 1, p.max_blocks * bs);
    for (int t0 = 0; t0 < nkeys; t0 += 64) {
        const int tk = t0 + lane;
        float score = -INFINITY;
        int64_t roff = -1;
        if (tk < nkeys) {
            const int64_t pb = table[tk / bs];
            if (pb >= 0 && pb < p.total_blocks) {
                roff = (pb * bs + tk % bs) * row_elems + static_cast<int64_t>(kvh) * HD;
                float dot = 0.0f;
                for (int d = 0; d < HD; ++d) dot = fmaf(q_s[d], bf16_to_f32(p.k[roff + d]), dot);
                score = dot;
            }
        }
        const float mn = fmaxf(m, wave_max(score));
        const float ms = mn == -INFINITY ? 0.0f : mn;
        const float alpha = fast_exp2(m - ms);
        const float pp = fast_exp2(score - ms);
        l = l * alpha + wave_sum(pp);
        m = mn;
#pragma unroll
        for (int k = 0; k < DPL; ++k) acc[k] *= alpha;
        p_s[lane] = pp;
        row_s[lane] = roff;
        __syncthreads();
        const int cnt = min(64, nkeys - t0);
        for (int jj = 0; jj < cnt; ++jj) {
            const int64_t vr = row_s[jj];
            if (vr < 0) continue;
            const float pj = p_s[jj];
#pragma unroll
            for (int k = 0; k < DPL; ++k) {
                const int d = lane + 64 * k;
                if (d < HD) acc[k] = fmaf(pj, bf16_to_f32(p.v[vr + d]), acc[k]);
            }
        }
        __syncthreads();
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    float* o = p.out + (static_cast<int64_t>(tokg) * p.Hq + h) * HD;
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
        const int d = lane + 64 * k;
        if (d < HD) o[d] = acc[k] * inv;
    }
}

template <int HD, int G, bool QF32>
int launch_prefill_shape(const PrefillParams& p, unsigned grid, hipStream_t s) {
    const size_t lds = PrefillLds<HD>::TOTAL + sizeof(int) * (static_cast<size_t>(p.B) + 3);
    auto kern = prefill_mfma_kernel<HD, G, QF32>;
    static size_t granted = 0;   // largest dynamic LDS size requested so far
    if (lds > granted) {
        SKV_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        granted = lds;
    }
    kern<<<grid, 64 * kPrefillWaves, lds, s>>>(p);
    return check_launch("prefill_mfma_kernel");
}

template <bool QF32>
int launch_prefill_mfma(PrefillParams p, int num_tokens, hipStream_t s) {
    const int G = p.Hq / p.Hkv;
    p.tile_tokens = kPrefillRows / G;
    const unsigned tiles = static_cast<unsigned>(cdiv(num_tokens, p.tile_tokens) + p.B);
    const unsigned grid = tiles * static_cast<unsigned>(p.Hkv);
#define SKV_PF(HD_, G_) \
    if (p.HD == HD_ && G == G_) return launch_prefill_shape<HD_, G_, QF32>(p, grid, s);
    SKV_PF(64, 1) SKV_PF(64, 2) SKV_PF(64, 4) SKV_PF(64, 8) SKV_PF(64, 16)
    SKV_PF(128, 1) SKV_PF(128, 2) SKV_PF(128, 4) SKV_PF(128, 8) SKV_PF(128, 16)
#undef SKV_PF
    return set_error(SKV_ERR_UNSUPPORTED, "no MFMA prefill kernel for head_dim %d, group %d", p.HD, G);
}

}  // namespace skv

using namespace skv;

extern "C" int skv_paged_prefill(const void* q, int q_dtype, const uint16_t* k_pool,
                                 const uint16_t* v_pool, int64_t total_blocks,
                                 const int32_t* block_tables, int max_blocks_per_seq,
                                 const int32_t* seq_offsets, const int32_t* context_lens,
                                 int num_seqs, int num_tokens, int num_q_heads, int num_kv_heads,
                                 int head_dim, int block_size, float scale, float* out,
                                 void* stream) {
    SKV_REQUIRE(q && k_pool && v_pool && block_tables && seq_offsets && context_lens && out,
                "skv_paged_prefill: NULL pointer");
    SKV_REQUIRE(q_dtype == SKV_DTYPE_BF16 || q_dtype == SKV_DTYPE_FP32,
                "skv_paged_prefill: unknown query dtype %d", q_dtype);
    SKV_REQUIRE(num_seqs > 0 && num_tokens >= 0 && num_q_heads > 0 && num_kv_heads > 0 &&
                    head_dim > 0 && block_size > 0 && total_blocks > 0 && max_blocks_per_seq > 0,
                "skv_paged_prefill: invalid dimensions");
    SKV_REQUIRE(num_q_heads % num_kv_heads == 0,
                "skv_paged_prefill: num_q_heads %d is not a multiple of num_kv_heads %d",
                num_q_heads, num_kv_heads);
    SKV_REQUIRE(scale > 0.0f && std::isfinite(scale), "skv_paged_prefill: scale must be positive and finite");
    SKV_REQUIRE(num_seqs <= kPrefillMaxBatch, "skv_paged_prefill: more than %d sequences per call",
                kPrefillMaxBatch);
    if (head_dim > 512)
        return set_error(SKV_ERR_UNSUPPORTED, "skv_paged_prefill: head_dim %d exceeds 512", head_dim);
    if (num_tokens == 0) return SKV_OK;
    PrefillParams p{};
    p.q = q;
    p.k = k_pool;
    p.v = v_pool;
    p.total_blocks = total_blocks;
    p.tables = block_tables;
    p.max_blocks = max_blocks_per_seq;
    p.offsets = seq_offsets;
    p.lens = context_lens;
    p.B = num_seqs;
    p.Hq = num_q_heads;
    p.Hkv = num_kv_heads;
    p.HD = head_dim;
    p.bs = block_size;
    p.qscale = scale * 1.4426950408889634f;
    p.out = out;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int G = num_q_heads / num_kv_heads;
    const bool mfma = block_size == 16 && (head_dim == 64 || head_dim == 128) &&
                      (G == 1 || G == 2 || G == 4 || G == 8 || G == 16) && aligned16(k_pool) &&
                      aligned16(v_pool) && aligned16(q) && aligned16(out);
    if (mfma)
        return q_dtype == SKV_DTYPE_FP32 ? launch_prefill_mfma<true>(p, num_tokens, s)
                                         : launch_prefill_mfma<false>(p, num_tokens, s);
    const unsigned grid = static_cast<unsigned>(num_tokens) * static_cast<unsigned>(num_q_heads);
    if (q_dtype == SKV_DTYPE_FP32)
        prefill_generic_kernel<true><<<grid, 64, 0, s>>>(p, num_tokens);
    else
        prefill_generic_kernel<false><<<grid, 64, 0, s>>>(p, num_tokens);
    return check_launch("prefill_generic_kernel");
}
