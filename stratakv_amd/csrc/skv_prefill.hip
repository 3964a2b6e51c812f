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
// * A workgroup of 4 wavefronts owns 64 query rows = the G heads of one kv
//   head for 64/G consecutive tokens of one sequence; wavefront w owns rows
//   16w..16w+15 (row r = token * G + head).  Every K/V byte staged in LDS is
//   used by all 64 rows.
// * Keys are walked 32 at a time (two 16-token blocks) up to the tile's last
//   position.  The workgroup stages K row-major (16-byte chunks XOR-swizzled
//   by row) and V transposed (Vt[dim][key], padded rows) in LDS; the next
//   step's K/V are loaded into registers while the current one is computed.
// * S^T = K Q^T on the matrix cores (v_mfma_f32_16x16x32_bf16: keys as rows,
//   query rows as columns), so each lane holds 8 scores of ONE query row
//   (column lane % 16): the causal/validity mask, the row max (2 shuffles)
//   and the rescale of that row's output are lane-local.
// * O^T += Vt P^T, also on the matrix cores: P goes from the S^T output
//   straight into the B operand (bf16, 8 keys per lane) with the key order
//   {4j..4j+3, 16+4j..16+4j+3} of lane group j, and the A operand reads Vt in
//   the same key order, so no shuffle or LDS round trip is needed for P.  P is
//   split into hi + lo bf16 parts (two MFMAs) so the P.V products keep ~16
//   mantissa bits, like the fp32 loops of the reference.
// * Online softmax in the exp2 domain with lazy rescaling (threshold 2^8).
// Other shapes run a simple kernel (one wavefront per token and query head).
#include "skv_common.h"

#include <algorithm>
#include <cmath>

namespace skv {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
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
// wavefront 0 (the same scan for every workgroup); returns the total.
__device__ int prefill_tile_scan(const PrefillParams& p, int* T_s) {
    const int lane = threadIdx.x;
    if (lane < 64) {
        int carry = 0;
        for (int b0 = 0; b0 < p.B; b0 += 64) {
            const int b = b0 + lane;
            int v = b < p.B ? cdiv(chunk_tokens(p, b), p.tile_tokens) : 0;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int u = __shfl_up(v, o, 64);
                if (lane >= o) v += u;
            }
            if (b < p.B) T_s[b + 1] = carry + v;
            carry += __shfl(v, 63, 64);
        }
        if (lane == 0) T_s[0] = 0;
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
// B operand: query row t, chunk 4cc + j; S^T output: keys 4j + i (+16 kt),
// query row t.  P^T B operand: query row t, keys {4j..4j+3, 16+4j..16+4j+3};
// Vt A operand: dim 16 dt + t, the same 8 keys; O^T output: dims 16 dt + 4j
// + i, query row t.
// ---------------------------------------------------------------------------
template <int HD, int G, bool QF32>
__global__ __launch_bounds__(256) void prefill_mfma_kernel(PrefillParams p) {
    constexpr int KS = 32;                  // keys per step (two blocks)
    constexpr int CH = HD / 8;              // 16-byte chunks per row
    constexpr int NMF = HD / 32;            // MFMAs per 16 keys for S
    constexpr int NDT = HD / 16;            // 16-dim tiles of O
    constexpr int QP = QF32 ? 2 : 1;
    constexpr int QT = 64 / G;              // tokens per tile
    constexpr int VS = KS + 4;              // Vt row stride (bf16): 72 bytes
    constexpr int LOADS = KS * CH / 256;    // 16-byte chunks per thread per step (K, and V)
    static_assert(LOADS >= 1 && KS * CH % 256 == 0, "load split");

    extern __shared__ int T_s[];            // [B + 1] tile prefix
    __shared__ u32x4_t k_s[KS * CH];        // K: row R, chunk c at R*CH + (c ^ swz(R))
    __shared__ uint16_t vt_s[HD * VS];      // V transposed: [dim][key]
    // Swizzle of K's 16-byte chunks by row so the 16 rows an MFMA operand read
    // touches (one chunk column) fall in 16 different bank groups.
    auto swz = [](int R) { return CH == 16 ? (R & 15) : ((R >> 1) & 7); };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t = lane & 15, j = lane >> 4;
    const int kvh = blockIdx.x % p.Hkv;
    const int tile = blockIdx.x / p.Hkv;

    const int ntiles = prefill_tile_scan(p, T_s);
    if (tile >= ntiles) return;
    const int b = find_tile_seq(T_s, p.B, tile);
    const int n = chunk_tokens(p, b);
    const int L = p.lens[b];
    const int tok0 = (tile - T_s[b]) * QT;             // first chunk token of the tile
    const int ntok = min(QT, n - tok0);
    const int base_pos = L - n + tok0;                 // position of the tile's first token
    const int last_pos = base_pos + ntok - 1;
    const int nb_seq = min(cdiv(max(L, 0), 16), p.max_blocks);
    const int keys_end = min(last_pos + 1, nb_seq * 16);  // keys [0, keys_end) may be read
    const int32_t* table = p.tables + static_cast<int64_t>(b) * p.max_blocks;
    const int64_t row_stride = static_cast<int64_t>(p.Hkv) * HD;

    // This lane's query row (column t of the S^T tiles).
    const int r = wv * 16 + t;
    const int qtok = r / G, qhead = kvh * G + (r % G);
    const bool row_live = qtok < ntok;
    const int qpos = row_live ? base_pos + qtok : -1;  // -1: every key masked
    const int64_t qrow = static_cast<int64_t>(p.offsets[b] + tok0 + qtok) * p.Hq + qhead;

    bf16x8_t qop[QP][NMF];
#pragma unroll
    for (int cc = 0; cc < NMF; ++cc) {
        u32x4_t hi = {0u, 0u, 0u, 0u}, lo = {0u, 0u, 0u, 0u};
        if (row_live) {
            const int64_t off = qrow * HD + (4 * cc + j) * 8;
            if constexpr (QF32) {
                const float4* qp = reinterpret_cast<const float4*>(static_cast<const float*>(p.q) + off);
                const float4 a0 = qp[0], a1 = qp[1];
                const float x[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                uint32_t hb[8], lb[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    hb[e] = f32_to_bf16_bits(x[e]);
                    lb[e] = f32_to_bf16_bits(x[e] - __uint_as_float(hb[e] << 16));
                }
                hi = u32x4_t{hb[0] | hb[1] << 16, hb[2] | hb[3] << 16, hb[4] | hb[5] << 16, hb[6] | hb[7] << 16};
                lo = u32x4_t{lb[0] | lb[1] << 16, lb[2] | lb[3] << 16, lb[4] | lb[5] << 16, lb[6] | lb[7] << 16};
            } else {
                hi = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p.q) + off);
            }
        }
        qop[0][cc] = __builtin_bit_cast(bf16x8_t, hi);
        if constexpr (QF32) qop[QP - 1][cc] = __builtin_bit_cast(bf16x8_t, lo);
    }

    // Loader mapping: thread -> (key row lr, chunk lc) for each of LOADS passes;
    // 16 consecutive threads read one 256-byte (HD 128) row slice.  `valid`
    // (the same in every thread) has bit k set when key k0 + k exists: below
    // keys_end and in a block whose table entry is inside the pool.
    auto load_step = [&](int k0, u32x4_t (&kr)[LOADS], u32x4_t (&vr)[LOADS], uint32_t& valid) {
        valid = 0;
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            const int kb = k0 + 16 * hb;
            if (kb < keys_end) {
                const int64_t pb = table[kb >> 4];
                if (pb >= 0 && pb < p.total_blocks) {
                    const int cnt = min(16, keys_end - kb);
                    valid |= (cnt == 16 ? 0xFFFFu : ((1u << cnt) - 1u)) << (16 * hb);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < LOADS; ++u) {
            const int idx = tid + 256 * u;
            const int lr = idx / CH, lc = idx % CH;
            kr[u] = u32x4_t{0u, 0u, 0u, 0u};
            vr[u] = u32x4_t{0u, 0u, 0u, 0u};
            if ((valid >> lr) & 1u) {
                const int key = k0 + lr;
                const int64_t pb = table[key >> 4];
                const int64_t off = (pb * 16 + (key & 15)) * row_stride + static_cast<int64_t>(kvh) * HD + lc * 8;
                kr[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p.k + off));
                vr[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p.v + off));
            }
        }
    };
    // Rows of keys that do not exist are stored as zeros (V must not carry
    // NaN from unused slots into 0 * V).
    auto store_step = [&](const u32x4_t (&kr)[LOADS], const u32x4_t (&vr)[LOADS]) {
#pragma unroll
        for (int u = 0; u < LOADS; ++u) {
            const int idx = tid + 256 * u;
            const int lr = idx / CH, lc = idx % CH;
            k_s[lr * CH + (lc ^ swz(lr))] = kr[u];
            const uint32_t w[4] = {vr[u].x, vr[u].y, vr[u].z, vr[u].w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                vt_s[(lc * 8 + e) * VS + lr] = static_cast<uint16_t>((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xFFFFu));
        }
    };

    f32x4_t acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY;   // reference max of this lane's row (log2 units)
    float lsum = 0.0f;     // this lane's share of the row's denominator

    const int nsteps = cdiv(keys_end, KS);
    u32x4_t kr[LOADS], vr[LOADS];
    uint32_t valid = 0, valid_next = 0;
    if (nsteps > 0) load_step(0, kr, vr, valid);
    for (int st = 0; st < nsteps; ++st) {
        __syncthreads();                 // every wavefront is done with the previous tiles
        store_step(kr, vr);
        __syncthreads();
        const uint32_t kvalid = valid;
        if (st + 1 < nsteps) {           // the next step's loads are in flight during compute
            load_step((st + 1) * KS, kr, vr, valid_next);
            valid = valid_next;
        }

        // ---- S^T tiles (keys 16 kt + 4j + i, query row t)
        f32x4_t s[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            s[kt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            const int R = kt * 16 + t;
#pragma unroll
            for (int cc = 0; cc < NMF; ++cc) {
                const bf16x8_t a = __builtin_bit_cast(bf16x8_t, k_s[R * CH + ((4 * cc + j) ^ swz(R))]);
#pragma unroll
                for (int qp = 0; qp < QP; ++qp)
                    s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qop[qp][cc], s[kt], 0, 0, 0);
            }
        }
        float sc[8];
        const int k0 = st * KS;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kl = kt * 16 + 4 * j + i;
                const bool keep = ((kvalid >> kl) & 1u) && (k0 + kl <= qpos);
                sc[kt * 4 + i] = keep ? s[kt][i] * p.qscale : -INFINITY;
            }
        float mb = sc[0];
#pragma unroll
        for (int e = 1; e < 8; ++e) mb = fmaxf(mb, sc[e]);
        mb = fmaxf(mb, shfl_xor_f(mb, 16));
        mb = fmaxf(mb, shfl_xor_f(mb, 32));
        if (mb > m + kPrefillLazy) {     // per-lane: the row's state is lane-local
            const float alpha = m == -INFINITY ? 0.0f : fast_exp2(m - mb);
            m = mb;
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[dt][i] *= alpha;
        }
        const float ms = m == -INFINITY ? 0.0f : m;
        float pr[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            pr[e] = fast_exp2(sc[e] - ms);
            lsum += pr[e];
        }
        // P^T operand, hi + lo bf16 parts.
        uint32_t ph[8], pl[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            ph[e] = f32_to_bf16_bits(pr[e]);
            pl[e] = f32_to_bf16_bits(pr[e] - __uint_as_float(ph[e] << 16));
        }
        const bf16x8_t phi = __builtin_bit_cast(
            bf16x8_t, u32x4_t{ph[0] | ph[1] << 16, ph[2] | ph[3] << 16, ph[4] | ph[5] << 16, ph[6] | ph[7] << 16});
        const bf16x8_t plo = __builtin_bit_cast(
            bf16x8_t, u32x4_t{pl[0] | pl[1] << 16, pl[2] | pl[3] << 16, pl[4] | pl[5] << 16, pl[6] | pl[7] << 16});

        // ---- O^T += Vt P^T
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            const uint16_t* vrow = vt_s + (dt * 16 + t) * VS;
            const uint2 a0 = *reinterpret_cast<const uint2*>(vrow + 4 * j);
            const uint2 a1 = *reinterpret_cast<const uint2*>(vrow + 16 + 4 * j);
            const bf16x8_t a = __builtin_bit_cast(bf16x8_t, u32x4_t{a0.x, a0.y, a1.x, a1.y});
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, phi, acc[dt], 0, 0, 0);
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, plo, acc[dt], 0, 0, 0);
        }
    }

    // ---- output: O[row t][dims 16 dt + 4j + i] = acc / l
    float ltot = lsum + shfl_xor_f(lsum, 16);
    ltot += shfl_xor_f(ltot, 32);
    if (row_live) {
        const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
        float* o = p.out + qrow * HD;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
            *reinterpret_cast<float4*>(o + dt * 16 + 4 * j) =
                make_float4(acc[dt][0] * inv, acc[dt][1] * inv, acc[dt][2] * inv, acc[dt][3] * inv);
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

template <bool QF32>
int launch_prefill_mfma(PrefillParams p, int num_tokens, hipStream_t s) {
    const int G = p.Hq / p.Hkv;
    p.tile_tokens = 64 / G;
    const unsigned tiles = static_cast<unsigned>(cdiv(num_tokens, p.tile_tokens) + p.B);
    const unsigned grid = tiles * static_cast<unsigned>(p.Hkv);
    const size_t lds = sizeof(int) * (static_cast<size_t>(p.B) + 1);
#define SKV_PF(HD_, G_)                                                        \
    if (p.HD == HD_ && G == G_) {                                              \
        prefill_mfma_kernel<HD_, G_, QF32><<<grid, 256, lds, s>>>(p);          \
        return check_launch("prefill_mfma_kernel");                            \
    }
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
