// skv_decode.hip -- paged decode attention (one query token per sequence,
// grouped-query attention over bf16 K/V pools in 16-token blocks).
//
// Replaces paged_attention_decode_kernel / paged_attention_decode_cuda of the
// reference (src/cuda/gemm_cuda.cu:304-429, 915-935).  The reference runs one
// 256-thread block per query head of one sequence, so each K/V byte is read by
// all G = Hq/Hkv query heads of its group, and it accumulates P.V in global
// memory.  Here the work is organised for CDNA4:
//
// * Work = the (sequence, kv head, block) triples, flattened, and split evenly
//   over a fixed set of persistent wavefronts ("stream-K"; each wavefront
//   derives the split itself from a scan of the context lengths): no tail of
//   idle CUs, and a wavefront whose range covers a whole (sequence, kv head)
//   segment writes the final output; only segments cut by a range boundary
//   leave partial (max, sum, acc) triples for the merge kernel (log-sum-exp
//   rescale).  The wavefronts of one workgroup take neighbouring kv heads of
//   the same range, so one CU reads adjacent slices of every block row.
// * A wavefront serves all G query heads of a kv head from one read of K/V.
//   q.k^T runs on the matrix cores: v_mfma_f32_16x16x32_bf16 with the 16 tokens
//   of a block as rows and the G heads (zero-padded to 16) as columns; fp32
//   queries are split into hi + lo bf16 parts (two MFMAs) so the products stay
//   fp32-accurate.  P.V stays on the VALU in fp32.
// * K and V rows are read 16 bytes per lane, HD/8 lanes per 128/256-byte row
//   (fully coalesced).  K goes through a per-wave LDS tile, stored with its
//   16-byte chunks XOR-swizzled by row, and comes back in the MFMA operand
//   layout (one 16-byte chunk of one token per lane) without bank conflicts.
//   Each wavefront keeps a ring of NBUF blocks in registers: while one is
//   computed the next NBUF - 1 are in flight, and the block addresses come
//   from table entries preloaded 64 at a time (no dependent table load per
//   block).  The rows are read with buffer loads through a descriptor that
//   spans exactly one block, so a ring position past the segment reads
//   through a descriptor of size 0 (zeros, no memory traffic).  K/V are read
//   once per step, so the loads carry the non-temporal hint (streamed through
//   L2 without displacing reused lines), which on MI355X raises the
//   achievable rate of this pattern by ~10 %.
// * Online softmax in the exp2 domain with lazy rescaling: the running max is
//   only raised (and acc, sum rescaled) when a block's max exceeds it by more
//   than 2^8, which after the first blocks is rare; the result is exact since
//   numerator and denominator share the same reference max.
#include "skv_append.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <mutex>
#include <string>
#include <unordered_map>

namespace skv {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct DecodeParams {
    const void* q;
    const uint16_t* k;
    const uint16_t* v;
    int64_t total_blocks;
    const int32_t* tables;
    int max_blocks;
    const int32_t* lens;   // [B] on the device, or nullptr -> single_len
    int single_len;
    int B, Hq, Hkv, HD, bs;
    float qscale;          // softmax scale * log2(e)
    float* out;            // [B][Hq][HD]
    int Hseg;              // segments per sequence: Hkv (MFMA kernel) or Hq (generic kernel)
    int NH;                // query heads per segment: G or 1
    int ranges;            // block ranges; the grid is ranges * Hseg wavefronts
    int min_per;           // minimum blocks per range
    int paired;            // 1: two workgroups per CU, the second half of the grid the younger wavefront of each SIMD
    int32_t* plan;         // [5 + B + 1]: total, per, used ranges, half, per_b, P[0..B]
    float* ws_ml;          // [2 * ranges * Hseg][NH][2]  (reference max in log2 units, sum)
    float* ws_acc;         // [2 * ranges * Hseg][NH][HD] (unnormalised P.V)
    // Fused append (MFMA kernel only): the new token of sequence b, at position
    // lens[b] - 1, rows [B][Hkv][HD]; nullptr = no append.
    const void* k_new;
    const void* v_new;
    int kv_new_fp32;       // 1: fp32 rows, rounded to nearest-even; 0: bf16 bits
    uint16_t* k_pool_w;    // the pools again, writable (the new rows are stored)
    uint16_t* v_pool_w;
    int merge_cw;          // output columns per merge workgroup (a multiple of 64)
    int max_slots;         // (range, head group) pairs the workspace holds partials for
    int seg_cost;          // stream-K: blocks' worth of time charged per segment start (see WorkSplit)
};

constexpr int kMaxHeadDim = 512;
constexpr int kMaxWaves = 8192;      // bound on persistent wavefronts (workspace sizing)
constexpr int kMaxBatchPerLaunch = 4096;  // sequences per launch (LDS prefix table)
constexpr float kLazyRescale = 8.0f;
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer descriptor: 32-bit data format, no swizzle
constexpr int kLoadNonTemporal = 2;     // cache policy of the K/V loads: nt (read once per step)

__device__ __forceinline__ int seq_len(const DecodeParams& p, int b) {
    return p.lens != nullptr ? p.lens[b] : p.single_len;
}

__device__ __forceinline__ int seq_blocks(const DecodeParams& p, int b) {
    const int L = seq_len(p, b);
    if (L <= 0) return 0;
    return std::min(cdiv(L, p.bs), p.max_blocks);
}

// ---------------------------------------------------------------------------
// Work split ("stream-K" over blocks).  Every workgroup builds P[b] = blocks of
// the sequences before b in LDS (a wave scan over the batch), so no planner
// launch is needed.  The flattened (sequence, block) space [0, P[B]) is cut
// into `used` ranges; wavefront w serves range w / Hseg for head group
// w % Hseg, so the Hseg wavefronts reading the head slices of the same
// 16-token blocks run side by side.  A segment = (sequence, head group): it is
// final when one range holds all of it; otherwise each range touching it
// leaves a partial in slot (2 * range + tail) * Hseg + group, tail = 1 when
// the segment starts strictly inside the range (then it is the range's last
// segment), 0 otherwise (the range's first segment).
//
// A segment start costs a wavefront about a memory round trip more than a
// block (finalising the previous segment, then the new segment's queries and
// table entries before its first K/V loads): per-wave timestamps of cfg3 on
// MI355X showed the ranges that cross a segment boundary ending ~4.3 us (~3.4
// blocks' time) after the others, and making most of the last ones.  So the
// split is over a "virtual" space in which every non-empty segment occupies
// seg_cost empty slots before its blocks: P_s holds that prefix, segment b's
// blocks sit at [seg_first(b), P_s[b + 1]), and a range that covers a segment
// start gets seg_cost fewer blocks.  The merge kernel reads the same prefix.
//
// Ranges [0, half) hold `per` blocks and ranges [half, used) `per_b`.  The
// split is even (half = used, per_b = per) unless the grid is paired: two
// workgroups per CU, two wavefronts per SIMD, where the second half of the
// grid is dispatched after the first and runs as the younger wavefront of
// every SIMD.  The SIMD issues for the older wavefront first, so with equal
// ranges the younger ones finished ~9 % later (per-wavefront timestamps, cfg3
// on MI355X); paired grids give the first half kPairShare / (kPairShare - 1)
// times the blocks of the second.
// ---------------------------------------------------------------------------
constexpr int kPairShare = 24;
constexpr int kSegmentCost = 4;  // seg_cost of the MFMA kernel's stream-K split

struct WorkSplit {
    int total, per, used, half, per_b;
    __device__ int lo(int r) const { return r <= half ? r * per : half * per + (r - half) * per_b; }
    __device__ int range_of(int pos) const {
        const int edge = half * per;
        return pos < edge ? pos / per : half + (pos - edge) / per_b;
    }
};

__device__ WorkSplit build_split(const DecodeParams& p, int* P_s, bool stream_k) {
    const int lane = threadIdx.x;
    if (lane < 64) {  // wavefront 0 of the workgroup scans
        int carry = 0;
        for (int b0 = 0; b0 < p.B; b0 += 64) {
            const int b = b0 + lane;
            int v = b < p.B ? seq_blocks(p, b) : 0;
            if (blockIdx.x == 0 && p.out != nullptr) {
                // Sequences without context produce zeros (workgroup 0 writes them).
                uint64_t empty = __ballot(b < p.B && v == 0);
                const int64_t row = static_cast<int64_t>(p.Hq) * p.HD;
                while (empty != 0) {
                    const int e = __builtin_ctzll(empty);
                    empty &= empty - 1;
                    float* o = p.out + static_cast<int64_t>(b0 + e) * row;
                    for (int64_t i = lane; i < row; i += 64) o[i] = 0.0f;
                }
            }
            if (v > 0) v += p.seg_cost;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int u = __shfl_up(v, o, 64);
                if (lane >= o) v += u;
            }
            if (b < p.B) P_s[b + 1] = carry + v;
            carry += __shfl(v, 63, 64);
        }
        if (lane == 0) P_s[0] = 0;
    }
    __syncthreads();
    WorkSplit ws{P_s[p.B], 0, 0, 0, 0};
    if (!stream_k) return ws;  // one workgroup per segment: no ranges
    ws.per = std::max(p.min_per, ws.total > 0 ? cdiv(ws.total, p.ranges) : 1);
    ws.used = ws.total > 0 ? cdiv(ws.total, ws.per) : 0;
    ws.half = ws.used;
    ws.per_b = ws.per;
    if (p.paired && ws.total > 0) {
        const int H = p.ranges / 2;
        const int pb = static_cast<int>(static_cast<int64_t>(ws.total) * (kPairShare - 1) /
                                        (static_cast<int64_t>(2) * kPairShare * H));
        const int pa = pb > 0 ? cdiv(ws.total - H * pb, H) : 0;
        if (pb >= p.min_per && pa >= pb) {
            ws.per = pa;
            ws.per_b = pb;
            ws.half = H;
            ws.used = H + cdiv(std::max(0, ws.total - H * pa), pb);
        }
    }
    if (blockIdx.x == 0 && lane < 64 && p.plan != nullptr) {  // publish for the merge kernel
        for (int i = lane; i <= p.B; i += 64) p.plan[5 + i] = P_s[i];
        if (lane == 0) {
            p.plan[0] = ws.total;
            p.plan[1] = ws.per;
            p.plan[2] = ws.used;
            p.plan[3] = ws.half;
            p.plan[4] = ws.per_b;
        }
    }
    return ws;
}

// Position of segment b's first block: past its seg_cost empty slots, unless
// it has no blocks.
__device__ __forceinline__ int seg_first(const int* P, int b, int seg_cost) {
    return P[b] + (P[b + 1] > P[b] ? seg_cost : 0);
}

// Sequence owning flattened block `pos`: P[b] <= pos < P[b+1].
__device__ __forceinline__ int find_seq(const int* P, int B, int pos) {
    int lo = 0, hi = B;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (P[mid] <= pos) lo = mid; else hi = mid;
    }
    return lo;
}

__device__ __forceinline__ int64_t partial_row(int range, bool tail, int Hseg, int group) {
    return (2 * static_cast<int64_t>(range) + (tail ? 1 : 0)) * Hseg + group;
}

// N values x (N = 8, 4, 2 or 1; o aligned to 4 N bytes) times sc.
template <int N>
__device__ __forceinline__ void store_scaled(float* o, const float* x, float sc) {
    if constexpr (N == 8) {
        reinterpret_cast<float4*>(o)[0] = make_float4(x[0] * sc, x[1] * sc, x[2] * sc, x[3] * sc);
        reinterpret_cast<float4*>(o)[1] = make_float4(x[4] * sc, x[5] * sc, x[6] * sc, x[7] * sc);
    } else if constexpr (N == 4) {
        *reinterpret_cast<float4*>(o) = make_float4(x[0] * sc, x[1] * sc, x[2] * sc, x[3] * sc);
    } else if constexpr (N == 2) {
        *reinterpret_cast<float2*>(o) = make_float2(x[0] * sc, x[1] * sc);
    } else {
        o[0] = x[0] * sc;
    }
}

// ---------------------------------------------------------------------------
// MFMA path: block_size 16, head_dim 64 or 128, G in {1, 2, 4, 8, 16}.
// Coalesced (V) layout: lane (r, c) = (lane / CH, lane % CH) holds rows
//   i*RPI + r (i < TPL) of a block, elements [8c, 8c + 8).
// MFMA layout: lane (t, j) = (lane % 16, lane / 16); the K operand of MFMA cc
//   is row t, chunk 4*cc + j, read from the LDS tile; the output holds
//   S[token 4j + i][head t].
// LDS tile: row R, chunk c stored at R*CH + (c ^ swz(R)), swz(R) = R for
//   CH = 16 and (R >> 1) & 7 for CH = 8, so the 16 lanes reading one chunk
//   column of 16 rows hit 16 distinct bank groups.
// Each wavefront owns its LDS tiles and synchronises only with itself
// (wave_lds_sync); the WPW wavefronts of a workgroup meet once, at the split.
// ---------------------------------------------------------------------------
// Wavefronts per SIMD the MFMA kernel is launched with (see launch_mfma_shape);
// also its register budget (launch bound).
constexpr int mfma_waves_per_simd(int HD, int G) { return HD == 64 && G < 16 ? 2 : 1; }

// SPLIT: short tables (at most WPW * NBUF blocks per sequence).  Workgroup
// = one (sequence, kv head) segment; its WPW wavefronts take consecutive
// sub-ranges of at most NBUF blocks, so every K/V load of the segment is in
// flight at once, and merge their partials through LDS (no merge launch).
template <int HD, int G, bool QF32, int WPW, int NBUF, bool SPLIT = false>
__global__ __launch_bounds__(64 * WPW, mfma_waves_per_simd(HD, G)) void decode_mfma_kernel(DecodeParams p) {
    constexpr int BS = 16;
    constexpr int CH = HD / 8;      // 16-byte chunks per row
    constexpr int RPI = 64 / CH;    // rows per coalesced load instruction
    constexpr int TPL = BS / RPI;   // rows per lane per block (coalesced layout)
    constexpr int NMF = HD / 32;    // MFMAs per block for q.k
    constexpr int QP = QF32 ? 2 : 1;
    static_assert(CH * RPI == 64 && RPI * TPL == BS && NMF * 4 == CH, "lane layout");
    static_assert(G >= 1 && G <= 16, "group size");

    // Per-wavefront LDS: the WPW wavefronts of a workgroup serve the same
    // range for WPW consecutive kv heads and only meet at the work split.
    extern __shared__ int P_s[];            // [B + 1] block prefix
    __shared__ u32x4_t k_all[WPW][BS * CH];  // one block of K for this kv head, swizzled
    __shared__ float p_all[WPW][BS * 16];    // probabilities [token][head]
    __shared__ float h_all[WPW][2][16];      // per-head (sum, max) at the end of a segment
    __shared__ float part_acc[SPLIT ? WPW : 1][SPLIT ? G * HD : 1];  // SPLIT: per-wave partials
    __shared__ float part_ml[SPLIT ? WPW : 1][2][16];

    const int wv = WPW == 1 ? 0 : __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    u32x4_t* k_s = k_all[wv];
    float* p_s = p_all[wv];
    float (*h_s)[16] = h_all[wv];
    const int r = lane / CH, c = lane % CH;
    const int t = lane & 15, j = lane >> 4;
    auto swz = [](int row) { return CH == 16 ? row : ((row >> 1) & 7); };
    const int Hkv = p.Hkv;
    const int w = blockIdx.x * WPW + wv;    // Hkv % WPW == 0: one range per workgroup
    const int kvh = SPLIT ? static_cast<int>(blockIdx.x % Hkv) : w % Hkv;
    const int range = w / Hkv;

    // SPLIT: the workgroup names its sequence, so the sequence's whole table
    // row (max_blocks <= 64 entries, one per lane) is loaded beside the
    // lengths, before the split is known: the block addresses then wait on one
    // dependent load (lengths and table together) instead of two.
    int trow = 0;
    if constexpr (SPLIT) {
        const int64_t row = static_cast<int64_t>(blockIdx.x / Hkv) * p.max_blocks;
        trow = p.tables[row + std::min(lane, p.max_blocks - 1)];
    }
    // Query chunks of head kvh * G + t (lanes t < G; zero for padded heads),
    // as loaded.  SPLIT knows its sequence here, so its queries are requested
    // with the table row and arrive by the split's barrier (one dependent
    // round trip less before the first K/V loads); stream-K loads them per
    // segment.
    float4 qa[NMF][2];
    u32x4_t qh[NMF];
    auto load_q_raw = [&](int bq) {
#pragma unroll
        for (int cc = 0; cc < NMF; ++cc) {
            qa[cc][0] = qa[cc][1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            qh[cc] = u32x4_t{0u, 0u, 0u, 0u};
            if (t < G) {
                const int64_t qoff = (static_cast<int64_t>(bq) * p.Hq + kvh * G + t) * HD + (4 * cc + j) * 8;
                if constexpr (QF32) {
                    const float4* qp = reinterpret_cast<const float4*>(static_cast<const float*>(p.q) + qoff);
                    qa[cc][0] = qp[0];
                    qa[cc][1] = qp[1];
                } else {
                    qh[cc] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p.q) + qoff);
                }
            }
        }
    };
    if constexpr (SPLIT) load_q_raw(static_cast<int>(blockIdx.x / Hkv));

    const WorkSplit split = build_split(p, P_s, !SPLIT);
    if (!SPLIT && range >= split.used) return;
    const int64_t row_stride = static_cast<int64_t>(Hkv) * HD;
    const int block_bytes = static_cast<int>(BS * row_stride * 2);
    int range_lo = SPLIT ? 0 : split.lo(range);
    int range_hi = SPLIT ? 0 : split.lo(range + 1);
    int b = 0;
    if constexpr (SPLIT) {
        // Wavefront wv: blocks [wv * NBUF, wv * NBUF + NBUF) of the segment.
        b = static_cast<int>(blockIdx.x / Hkv);
        range_lo = std::min(P_s[b] + wv * NBUF, P_s[b + 1]);
        range_hi = std::min(range_lo + NBUF, P_s[b + 1]);
    }
    int pos = range_lo;
    const int end = SPLIT ? range_hi : std::min(range_hi, split.total);
    if (!SPLIT) b = find_seq(P_s, p.B, pos);
    const int h0 = kvh * G;

    while (!SPLIT || pos < end) {
        const int seg_lo = SPLIT ? P_s[b] : seg_first(P_s, b, p.seg_cost), seg_hi = P_s[b + 1];
        if (!SPLIT) {  // the range may start among, or end within, the segment's empty slots
            if (end <= seg_lo) break;
            pos = std::max(pos, seg_lo);
        }
        const int nb = seg_hi - seg_lo;
        const int k0 = pos - seg_lo;
        const int stop = std::min(end, seg_hi);
        const int kb1 = stop - seg_lo;
        const int L = seq_len(p, b);
        const int Leff = std::min(L, nb * BS);
        const int32_t* table = p.tables + static_cast<int64_t>(b) * p.max_blocks;

        // Fused append: the wavefront whose range holds the segment's last block
        // takes the new token's K/V row (position L - 1, slot = row i_new * RPI
        // + r_new of that block): it replaces the pool's row in registers when
        // the block is consumed and is stored into the pool after the segment.
        // Skipped, like skv_kv_append, when the position is beyond the table or
        // its block is outside the pool.
        int kb_new = -1, i_new = 0, r_new = 0;
        int64_t new_dst = 0;
        u32x4_t knew = {0u, 0u, 0u, 0u}, vnew = {0u, 0u, 0u, 0u};
        if (p.k_new != nullptr && kb1 == nb && L >= 1 && L <= nb * BS) {
            const int64_t e = SPLIT ? __shfl(trow, nb - 1, 64) : table[nb - 1];
            if (e >= 0 && e < p.total_blocks) {
                const int slot = (L - 1) - (nb - 1) * BS;
                kb_new = nb - 1;
                i_new = slot / RPI;
                r_new = slot % RPI;
                new_dst = (e * BS + slot) * row_stride + static_cast<int64_t>(kvh) * HD + c * 8;
                if (r == r_new) {
                    const int64_t src = (static_cast<int64_t>(b) * Hkv + kvh) * HD + c * 8;
                    if (p.kv_new_fp32) {
                        const float4* ks = reinterpret_cast<const float4*>(static_cast<const float*>(p.k_new) + src);
                        const float4* vs = reinterpret_cast<const float4*>(static_cast<const float*>(p.v_new) + src);
                        const float4 k0 = ks[0], k1 = ks[1], v0 = vs[0], v1 = vs[1];
                        knew = u32x4_t{pack_bf16x2(k0.x, k0.y), pack_bf16x2(k0.z, k0.w),
                                       pack_bf16x2(k1.x, k1.y), pack_bf16x2(k1.z, k1.w)};
                        vnew = u32x4_t{pack_bf16x2(v0.x, v0.y), pack_bf16x2(v0.z, v0.w),
                                       pack_bf16x2(v1.x, v1.y), pack_bf16x2(v1.z, v1.w)};
                    } else {
                        knew = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p.k_new) + src);
                        vnew = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p.v_new) + src);
                    }
                }
            }
        }

        // q operand(s): head h0 + t, chunk 4*cc + j; zero for padded heads.
        if constexpr (!SPLIT) load_q_raw(b);
        bf16x8_t qop[QP][NMF];
#pragma unroll
        for (int cc = 0; cc < NMF; ++cc) {
            u32x4_t hi = qh[cc], lo = {0u, 0u, 0u, 0u};
            if constexpr (QF32) {
                const float4 a0 = qa[cc][0], a1 = qa[cc][1];
                const float x[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                uint32_t hb[8], lb[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    hb[e] = f32_to_bf16_bits(x[e]);
                    lb[e] = f32_to_bf16_bits(x[e] - __uint_as_float(hb[e] << 16));
                }
                hi = u32x4_t{hb[0] | hb[1] << 16, hb[2] | hb[3] << 16, hb[4] | hb[5] << 16, hb[6] | hb[7] << 16};
                lo = u32x4_t{lb[0] | lb[1] << 16, lb[2] | lb[3] << 16, lb[4] | lb[5] << 16, lb[6] | lb[7] << 16};
            }
            qop[0][cc] = __builtin_bit_cast(bf16x8_t, hi);
            if constexpr (QF32) qop[QP - 1][cc] = __builtin_bit_cast(bf16x8_t, lo);
        }

        float m = -INFINITY;   // reference max of head t (log2 units), equal across j
        float lpart = 0.0f;    // sum of this lane's probabilities for head t
        float acc[G][8];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;

        const int lane_off_b = static_cast<int>((r * row_stride + static_cast<int64_t>(kvh) * HD + c * 8) * 2);

        // Table entries of the segment, 64 at a time: lane i holds entry tb + i
        // (tv) and tb + 64 + i (tvn, loaded one chunk ahead), so the block
        // addresses never wait on a dependent table load.
        auto table_entry = [&](int k) -> int {
            const int kc = k < kb1 ? k : kb1 - 1;
            if constexpr (SPLIT) return __shfl(trow, kc, 64);  // kc < nb <= max_blocks
            return table[kc];
        };
        int tb = k0;
        int tv = table_entry(tb + lane);
        int tvn = table_entry(tb + 64 + lane);

        // Loads of block kb into one register buffer.  Every call issues the
        // same loads, so the compiler's wait counts stay exact: a position
        // past the segment, or a table entry outside the pool, reads through
        // a buffer descriptor of size 0, whose loads return zeros without
        // touching memory.  The return value says whether the block is real.
        auto issue = [&](int kb, u32x4_t (&kk)[TPL], u32x4_t (&vv)[TPL]) -> bool {
            const bool in_seg = kb < kb1;
            kb = in_seg ? kb : kb1 - 1;
            if (kb - tb >= 64) {  // blocks are issued in order: advance one chunk
                tb += 64;
                tv = tvn;
                tvn = table_entry(tb + 64 + lane);
            }
            const int64_t e = __builtin_amdgcn_readlane(tv, kb - tb);
            const bool valid = in_seg && e >= 0 && e < p.total_blocks;
            const int64_t base = (valid ? e : 0) * BS * row_stride;
            const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<uint16_t*>(p.k + base), 0, valid ? block_bytes : 0, kRsrcWord3);
            const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<uint16_t*>(p.v + base), 0, valid ? block_bytes : 0, kRsrcWord3);
#pragma unroll
            for (int i = 0; i < TPL; ++i) {
                const int soff = static_cast<int>(i * RPI * row_stride * 2);
                kk[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, lane_off_b, soff, kLoadNonTemporal));
                vv[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, lane_off_b, soff, kLoadNonTemporal));
            }
            return valid;
        };

        auto consume = [&](int kb, u32x4_t (&kk)[TPL], u32x4_t (&vv)[TPL]) {
            if (kb == kb_new) {  // the block that receives the appended token
#pragma unroll
                for (int i = 0; i < TPL; ++i) {
                    if (i == i_new && r == r_new) {
                        kk[i] = knew;
                        vv[i] = vnew;
                    }
                }
            }
            // ---- K through the LDS tile into the MFMA operand layout
#pragma unroll
            for (int i = 0; i < TPL; ++i) {
                const int row = i * RPI + r;
                k_s[row * CH + (c ^ swz(row))] = kk[i];
            }
            wave_lds_sync();
            // ---- scores S[token 4j+i][head t] on the matrix cores
            f32x4_t sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int cc = 0; cc < NMF; ++cc) {
                const bf16x8_t a = __builtin_bit_cast(bf16x8_t, k_s[t * CH + ((4 * cc + j) ^ swz(t))]);
#pragma unroll
                for (int qp = 0; qp < QP; ++qp)
                    sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qop[qp][cc], sacc, 0, 0, 0);
            }
            const int tok = kb * BS + 4 * j;
            float s[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) s[i] = tok + i < Leff ? sacc[i] * p.qscale : -INFINITY;
            float mb = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
            // (ds_bpermute: on the LDS pipe beside the VALU work of the block,
            // measurably faster here than the VALU permlane swaps)
            mb = fmaxf(mb, shfl_xor_f(mb, 16));
            mb = fmaxf(mb, shfl_xor_f(mb, 32));

            // ---- lazy rescale (wave-uniform branch)
            const bool need = mb > m + kLazyRescale;
            if (__any(need)) {
                const float mn = need ? mb : m;
                // Before the first block m = -inf and acc, sum are 0: factor 0.
                const float alpha = m == -INFINITY ? 0.0f : fast_exp2(m - mn);
                m = mn;
                lpart *= alpha;
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float a = lane_value(alpha, g);  // lane g holds head g
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[g][e] *= a;
                }
            }
            const float ms = m == -INFINITY ? 0.0f : m;
            float pr[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) pr[i] = fast_exp2(s[i] - ms);
            lpart += (pr[0] + pr[1]) + (pr[2] + pr[3]);
            if (t < G) {
#pragma unroll
                for (int i = 0; i < 4; ++i) p_s[(4 * j + i) * 16 + t] = pr[i];
            }
            wave_lds_sync();

            // ---- P.V on the VALU (coalesced V layout)
            const bool tail = kb * BS + BS > Leff;
#pragma unroll
            for (int i = 0; i < TPL; ++i) {
                const int row = i * RPI + r;
                u32x4_t vw = vv[i];
                if (tail && kb * BS + row >= Leff) vw = u32x4_t{0u, 0u, 0u, 0u};
                float vf[8];
                vf[0] = bf16_lo(vw.x); vf[1] = bf16_hi(vw.x);
                vf[2] = bf16_lo(vw.y); vf[3] = bf16_hi(vw.y);
                vf[4] = bf16_lo(vw.z); vf[5] = bf16_hi(vw.z);
                vf[6] = bf16_lo(vw.w); vf[7] = bf16_hi(vw.w);
                float pv[G];
#pragma unroll
                for (int g = 0; g < G; ++g) pv[g] = p_s[row * 16 + g];
#pragma unroll
                for (int g = 0; g < G; ++g)
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(pv[g], vf[e], acc[g][e]);
            }
            wave_lds_sync();
        };

        // Ring of NBUF register buffers, unrolled so that buffer u always
        // holds block kb + u: while one block is consumed the next NBUF - 1
        // are in flight, and no register copy forces an early wait.
        u32x4_t kbuf[NBUF][TPL], vbuf[NBUF][TPL];
        bool okb[NBUF];
#pragma unroll
        for (int u = 0; u < NBUF; ++u) okb[u] = issue(k0 + u, kbuf[u], vbuf[u]);
        for (int kb = k0; kb < kb1; kb += NBUF) {
#pragma unroll
            for (int u = 0; u < NBUF; ++u) {
                if (okb[u]) consume(kb + u, kbuf[u], vbuf[u]);
                okb[u] = issue(kb + u + NBUF, kbuf[u], vbuf[u]);
            }
        }

        if (kb_new >= 0 && r == r_new) {  // fused append: store the new row
            *reinterpret_cast<u32x4_t*>(p.k_pool_w + new_dst) = knew;
            *reinterpret_cast<u32x4_t*>(p.v_pool_w + new_dst) = vnew;
        }

        // ---- finalise the segment: sum the row groups by a reduce-scatter,
        // after which lane (r, c) holds NF consecutive (head, element) values
        // v = NF * r + i (head v / 8, dims 8c + v % 8), exactly what it stores.
        constexpr int NV = G * 8;
        constexpr int LO = CH == 8 ? 3 : 4;
        constexpr int NF = NV >> (6 - LO);
        float v[NV];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) v[g * 8 + e] = acc[g][e];
        reduce_scatter_high_bits<NV, LO>(v);
        const float ltot = xor32_sum(xor16_sum(lpart));
        if (j == 0) {
            h_s[0][t] = ltot;
            h_s[1][t] = m;
        }
        wave_lds_sync();
        const bool final_out = !SPLIT && seg_lo >= range_lo && seg_hi <= range_hi;
        const int64_t prow = partial_row(range, seg_lo > range_lo, Hkv, kvh);
        // Lane (r, c) stores VPH values of each of its NHL heads at dims d0...
        constexpr int NHL = NF >= 8 ? NF / 8 : 1;
        constexpr int VPH = NF >= 8 ? 8 : NF;
        const int g0 = NF * r / 8;
        const int d0 = 8 * c + (NF >= 8 ? 0 : NF * r % 8);
        const bool owns_ml = c == 0 && d0 == 0;  // one lane per head stores (max, sum)
#pragma unroll
        for (int hh = 0; hh < NHL; ++hh) {
            const int g = g0 + hh;
            const float lsum = h_s[0][g];
            const float* x = v + VPH * hh;
            if (final_out) {
                store_scaled<VPH>(p.out + (static_cast<int64_t>(b) * p.Hq + h0 + g) * HD + d0, x,
                                  lsum > 0.0f ? 1.0f / lsum : 0.0f);
            } else if constexpr (SPLIT) {  // this wavefront's LDS slot
                store_scaled<VPH>(&part_acc[wv][g * HD + d0], x, 1.0f);
                if (owns_ml) {
                    part_ml[wv][0][g] = h_s[1][g];
                    part_ml[wv][1][g] = lsum;
                }
            } else {  // workspace slot, merged by decode_merge_kernel
                store_scaled<VPH>(p.ws_acc + (prow * G + g) * HD + d0, x, 1.0f);
                if (owns_ml)
                    *reinterpret_cast<float2*>(p.ws_ml + (prow * G + g) * 2) = make_float2(h_s[1][g], lsum);
            }
        }

        wave_lds_sync();

        pos = stop;
        if (SPLIT || pos >= end) break;
        do {
            ++b;
        } while (P_s[b + 1] == P_s[b]);
    }

    if constexpr (SPLIT) {
        // Merge the WPW sub-range partials of the segment (wavefronts past the
        // segment's last sub-range hold none):
        //   out = sum_w acc_w 2^(m_w - M) / sum_w l_w 2^(m_w - M),  M = max_w m_w.
        const int nw = std::min(WPW, cdiv(P_s[b + 1] - P_s[b], NBUF));
        __syncthreads();
        float* out0 = p.out + (static_cast<int64_t>(b) * p.Hq + h0) * HD;
        for (int col = threadIdx.x; col < G * HD; col += 64 * WPW) {
            const int g = col / HD;
            float M = -INFINITY;
            for (int u = 0; u < nw; ++u) M = fmaxf(M, part_ml[u][0][g]);
            float L = 0.0f, A = 0.0f;
            if (M != -INFINITY) {
                for (int u = 0; u < nw; ++u) {
                    const float wgt = fast_exp2(part_ml[u][0][g] - M);
                    L = fmaf(wgt, part_ml[u][1][g], L);
                    A = fmaf(wgt, part_acc[u][col], A);
                }
            }
            if (nw > 0) out0[col] = L > 0.0f ? A / L : 0.0f;
        }
    }
}

// ---------------------------------------------------------------------------
// Load-pattern calibration: the MFMA decode kernel's K/V reads with the
// attention math replaced by a checksum.  Same work split (stream-K ranges
// over the flattened (sequence, block) space, WPW neighbouring kv heads per
// workgroup), same table preloading, same ring of NBUF blocks per wavefront
// and the same non-temporal buffer loads, issued in the same order; each
// consumed block is folded into a wrapping 32-bit sum of its K and V words.
// sums[b * Hkv + h] receives the sum over the sequence's seq_blocks(b) blocks
// (all 16 rows of each, the head-h slice of K and of V; a table entry outside
// the pool contributes 0), so the result checks that every block was read
// exactly once, whatever the split.  Its time is the rate the decode's
// loads alone reach on this device: the ceiling the decode kernel is measured
// against.
// ---------------------------------------------------------------------------
template <int HD, int WPW, int NBUF>
__global__ __launch_bounds__(64 * WPW) void block_stream_checksum_kernel(DecodeParams p, uint32_t* sums) {
    constexpr int BS = 16;
    constexpr int CH = HD / 8;
    constexpr int RPI = 64 / CH;
    constexpr int TPL = BS / RPI;
    extern __shared__ int P_s[];

    const int wv = WPW == 1 ? 0 : __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int r = lane / CH, c = lane % CH;
    const int Hkv = p.Hkv;
    const int w = blockIdx.x * WPW + wv;
    const int kvh = w % Hkv;
    const int range = w / Hkv;
    const WorkSplit split = build_split(p, P_s, true);
    if (range >= split.used) return;
    const int64_t row_stride = static_cast<int64_t>(Hkv) * HD;
    const int block_bytes = static_cast<int>(BS * row_stride * 2);
    const int range_lo = split.lo(range);
    const int end = std::min(split.lo(range + 1), split.total);
    int pos = range_lo;
    int b = find_seq(P_s, p.B, pos);
    const int lane_off_b = static_cast<int>((r * row_stride + static_cast<int64_t>(kvh) * HD + c * 8) * 2);

    while (true) {
        const int seg_lo = seg_first(P_s, b, p.seg_cost), seg_hi = P_s[b + 1];
        if (end <= seg_lo) break;
        pos = std::max(pos, seg_lo);
        const int k0 = pos - seg_lo;
        const int stop = std::min(end, seg_hi);
        const int kb1 = stop - seg_lo;
        const int32_t* table = p.tables + static_cast<int64_t>(b) * p.max_blocks;
        auto table_entry = [&](int k) -> int { return table[k < kb1 ? k : kb1 - 1]; };
        int tb = k0;
        int tv = table_entry(tb + lane);
        int tvn = table_entry(tb + 64 + lane);
        auto issue = [&](int kb, u32x4_t (&kk)[TPL], u32x4_t (&vv)[TPL]) -> bool {
            const bool in_seg = kb < kb1;
            kb = in_seg ? kb : kb1 - 1;
            if (kb - tb >= 64) {
                tb += 64;
                tv = tvn;
                tvn = table_entry(tb + 64 + lane);
            }
            const int64_t e = __builtin_amdgcn_readlane(tv, kb - tb);
            const bool valid = in_seg && e >= 0 && e < p.total_blocks;
            const int64_t base = (valid ? e : 0) * BS * row_stride;
            const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<uint16_t*>(p.k + base), 0, valid ? block_bytes : 0, kRsrcWord3);
            const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<uint16_t*>(p.v + base), 0, valid ? block_bytes : 0, kRsrcWord3);
#pragma unroll
            for (int i = 0; i < TPL; ++i) {
                const int soff = static_cast<int>(i * RPI * row_stride * 2);
                kk[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, lane_off_b, soff, kLoadNonTemporal));
                vv[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, lane_off_b, soff, kLoadNonTemporal));
            }
            return valid;
        };
        uint32_t acc = 0;
        auto consume = [&](u32x4_t (&kk)[TPL], u32x4_t (&vv)[TPL]) {
#pragma unroll
            for (int i = 0; i < TPL; ++i)
                acc += (kk[i].x + kk[i].y) + (kk[i].z + kk[i].w) + (vv[i].x + vv[i].y) + (vv[i].z + vv[i].w);
        };
        u32x4_t kbuf[NBUF][TPL], vbuf[NBUF][TPL];
        bool okb[NBUF];
#pragma unroll
        for (int u = 0; u < NBUF; ++u) okb[u] = issue(k0 + u, kbuf[u], vbuf[u]);
        for (int kb = k0; kb < kb1; kb += NBUF) {
#pragma unroll
            for (int u = 0; u < NBUF; ++u) {
                if (okb[u]) consume(kbuf[u], vbuf[u]);
                okb[u] = issue(kb + u + NBUF, kbuf[u], vbuf[u]);
            }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) acc += static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc), o, 64));
        if (lane == 0) atomicAdd(sums + static_cast<int64_t>(b) * Hkv + kvh, acc);

        pos = stop;
        if (pos >= end) break;
        do {
            ++b;
        } while (P_s[b + 1] == P_s[b]);
    }
}

// ---------------------------------------------------------------------------
// Generic path: any block size, head_dim <= 512, any group size.  Segments are
// (sequence, query head); lanes own tokens for q.k (q staged in LDS) and head
// dimensions for P.V.  Correct for every shape the reference accepts; the
// MFMA path covers the benchmark geometries.
// ---------------------------------------------------------------------------
template <bool QF32>
__global__ __launch_bounds__(64) void decode_generic_kernel(DecodeParams p) {
    constexpr int DPL = kMaxHeadDim / 64;
    extern __shared__ int P_s[];    // [B + 1] block prefix
    __shared__ float q_s[kMaxHeadDim];
    __shared__ float p_s[64];
    __shared__ int64_t row_s[64];

    const int lane = threadIdx.x;
    const int Hq = p.Hq, HD = p.HD, bs = p.bs;
    const int w = blockIdx.x;
    const int h = w % Hq;
    const int range = w / Hq;
    const WorkSplit split = build_split(p, P_s, true);
    if (range >= split.used) return;
    const int64_t row_elems = static_cast<int64_t>(p.Hkv) * HD;
    const int range_lo = split.lo(range);
    const int range_hi = split.lo(range + 1);
    int pos = range_lo;
    const int end = std::min(range_hi, split.total);
    int b = find_seq(P_s, p.B, pos);
    const int kvh = h / (Hq / p.Hkv);

    while (true) {
        const int seg_lo = P_s[b], seg_hi = P_s[b + 1];
        const int nb = seg_hi - seg_lo;
        const int k0 = pos - seg_lo;
        const int stop = std::min(end, seg_hi);
        const int kb1 = stop - seg_lo;
        const int L = seq_len(p, b);
        const int Leff = std::min(L, nb * bs);
        const int tok0 = k0 * bs;
        const int tok1 = std::min(kb1 * bs, Leff);
        const int32_t* table = p.tables + static_cast<int64_t>(b) * p.max_blocks;

        const int64_t qoff = (static_cast<int64_t>(b) * Hq + h) * HD;
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

        for (int t0 = tok0; t0 < tok1; t0 += 64) {
            const int tk = t0 + lane;
            float score = -INFINITY;
            int64_t roff = -1;
            if (tk < tok1) {
                const int64_t pb = table[tk / bs];
                if (pb >= 0 && pb < p.total_blocks) {
                    roff = (pb * bs + tk % bs) * row_elems + static_cast<int64_t>(kvh) * HD;
                    const uint16_t* kr = p.k + roff;
                    float dot = 0.0f;
                    for (int d = 0; d < HD; ++d) dot = fmaf(q_s[d], bf16_to_f32(kr[d]), dot);
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
            const int n = std::min(64, tok1 - t0);
            for (int jj = 0; jj < n; ++jj) {
                const int64_t vr = row_s[jj];
                if (vr < 0) continue;
                const float pj = p_s[jj];
                const uint16_t* vrow = p.v + vr;
#pragma unroll
                for (int k = 0; k < DPL; ++k) {
                    const int d = lane + 64 * k;
                    if (d < HD) acc[k] = fmaf(pj, bf16_to_f32(vrow[d]), acc[k]);
                }
            }
            __syncthreads();
        }

        const bool final_out = seg_lo >= range_lo && seg_hi <= range_hi;
        if (final_out) {
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            float* o = p.out + (static_cast<int64_t>(b) * Hq + h) * HD;
#pragma unroll
            for (int k = 0; k < DPL; ++k) {
                const int d = lane + 64 * k;
                if (d < HD) o[d] = acc[k] * inv;
            }
        } else {
            const int64_t row = partial_row(range, seg_lo > range_lo, Hq, h);
#pragma unroll
            for (int k = 0; k < DPL; ++k) {
                const int d = lane + 64 * k;
                if (d < HD) p.ws_acc[row * HD + d] = acc[k];
            }
            if (lane == 0) {
                p.ws_ml[row * 2 + 0] = m;
                p.ws_ml[row * 2 + 1] = l;
            }
        }
        __syncthreads();

        pos = stop;
        if (pos >= end) break;
        do {
            ++b;
        } while (P_s[b + 1] == P_s[b]);
    }
}

// ---------------------------------------------------------------------------
// Merge of the segments cut by range boundaries:
//   out = sum_r acc_r 2^(m_r - M) / sum_r l_r 2^(m_r - M),  M = max_r m_r,
// over the n ranges r that touch the segment, per query head.  One 256-thread
// workgroup per (segment, chunk of merge_cw output columns).  With at most
// kMergeFew partials (kMergeFew / 2 when a thread covers 4 columns; long and
// medium batches) every thread loads all the partials of its columns in one
// round.  With more (short batches, one long sequence), thread (c, pg) =
// (t % 64, t / 64) takes partials pg, pg + 4, ... of column c, 8 at a time
// with all their loads in flight, and keeps its own (max, sum, acc) triple,
// rescaled per batch; the 4 partial groups are combined the same way through
// LDS.  Segments held by one range, and sequences without context, were
// written by the attention kernel; with a single range the merge is not
// launched at all.
// ---------------------------------------------------------------------------
constexpr int kMergeFew = 16;   // partials merged in one round of loads

// NP partials (exactly), NC columns per thread: every load is unconditional,
// so all 3 * NP * NC of them are in flight together (a conditional load makes
// the compiler wait for it before issuing the next one).
template <int NC, int NP>
__device__ __forceinline__ void merge_few(const DecodeParams& p, int grp, int r0, bool first_tail,
                                          float* out0, int c0, int c1) {
    const int t = threadIdx.x;
    const int HD = p.HD, NH = p.NH;
    float a[NC][NP], m[NC][NP], l[NC][NP];
#pragma unroll
    for (int e = 0; e < NC; ++e) {
        const int col = min(c0 + t + 256 * e, c1 - 1);
        const int g = col / HD;
        const int d = col - g * HD;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int64_t row = partial_row(r0 + i, i == 0 && first_tail, p.Hseg, grp) * NH + g;
            a[e][i] = p.ws_acc[row * HD + d];
            m[e][i] = p.ws_ml[row * 2];
            l[e][i] = p.ws_ml[row * 2 + 1];
        }
    }
#pragma unroll
    for (int e = 0; e < NC; ++e) {
        const int col = c0 + t + 256 * e;
        if (col >= c1) continue;
        float M = -INFINITY;
#pragma unroll
        for (int i = 0; i < NP; ++i) M = fmaxf(M, m[e][i]);
        float L = 0.0f, A = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const float w = fast_exp2(m[e][i] - M);
                L = fmaf(w, l[e][i], L);
                A = fmaf(w, a[e][i], A);
            }
        }
        out0[col] = L > 0.0f ? A / L : 0.0f;
    }
}

template <int NC>
__device__ __forceinline__ void merge_few_n(const DecodeParams& p, int grp, int r0, int n,
                                            bool first_tail, float* out0, int c0, int c1) {
    switch (n) {
        case 2: merge_few<NC, 2>(p, grp, r0, first_tail, out0, c0, c1); break;
        case 3: merge_few<NC, 3>(p, grp, r0, first_tail, out0, c0, c1); break;
        case 4: merge_few<NC, 4>(p, grp, r0, first_tail, out0, c0, c1); break;
        case 5: merge_few<NC, 5>(p, grp, r0, first_tail, out0, c0, c1); break;
        case 6: merge_few<NC, 6>(p, grp, r0, first_tail, out0, c0, c1); break;
        case 7: merge_few<NC, 7>(p, grp, r0, first_tail, out0, c0, c1); break;
        case 8: merge_few<NC, 8>(p, grp, r0, first_tail, out0, c0, c1); break;
        default:
            if constexpr (NC <= 2) {
                switch (n) {
                    case 9: merge_few<NC, 9>(p, grp, r0, first_tail, out0, c0, c1); break;
                    case 10: merge_few<NC, 10>(p, grp, r0, first_tail, out0, c0, c1); break;
                    case 11: merge_few<NC, 11>(p, grp, r0, first_tail, out0, c0, c1); break;
                    case 12: merge_few<NC, 12>(p, grp, r0, first_tail, out0, c0, c1); break;
                    case 13: merge_few<NC, 13>(p, grp, r0, first_tail, out0, c0, c1); break;
                    case 14: merge_few<NC, 14>(p, grp, r0, first_tail, out0, c0, c1); break;
                    case 15: merge_few<NC, 15>(p, grp, r0, first_tail, out0, c0, c1); break;
                    default: merge_few<NC, 16>(p, grp, r0, first_tail, out0, c0, c1); break;
                }
            }
            break;
    }
}

__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeParams p) {
    __shared__ float gm[4], gl[4];
    __shared__ float ga[4][64];
    const int t = threadIdx.x;
    const int HD = p.HD, NH = p.NH;
    const int cols = NH * HD;
    const int cw = p.merge_cw;
    const int nchunk = cdiv(cols, cw);
    const int s = blockIdx.x / nchunk;
    const int chunk = blockIdx.x - s * nchunk;
    const int c0 = chunk * cw, c1 = min(cols, c0 + cw);
    const int b = s / p.Hseg;
    const int grp = s - b * p.Hseg;
    WorkSplit split;
    split.total = p.plan[0];
    split.per = p.plan[1];
    split.used = p.plan[2];
    split.half = p.plan[3];
    split.per_b = p.plan[4];
    const int32_t* P = p.plan + 5;
    const int lo = seg_first(P, b, p.seg_cost), hi = P[b + 1];
    float* out0 = p.out + (static_cast<int64_t>(b) * p.Hq + grp * NH) * HD;
    if (lo == hi) return;  // no context: zeroed by the attention kernel
    const int r0 = split.range_of(lo), r1 = split.range_of(hi - 1);
    if (r0 == r1) return;
    const int n = r1 - r0 + 1;
    const bool first_tail = lo > split.lo(r0);
    if ((n <= kMergeFew && cw <= 512) || (n <= kMergeFew / 2 && cw <= 1024)) {
        // Few partials (long and medium batches): thread t takes columns
        // c0 + t, c0 + t + 256, ... with all n partials of each loaded at once.
        if (cw <= 256) merge_few_n<1>(p, grp, r0, n, first_tail, out0, c0, c1);
        else if (cw <= 512) merge_few_n<2>(p, grp, r0, n, first_tail, out0, c0, c1);
        else merge_few_n<4>(p, grp, r0, n, first_tail, out0, c0, c1);
        return;
    }
    // Many partials (short batches, one long sequence): 64 columns at a time,
    // thread (c, pg) = (t % 64, t / 64) taking partials pg, pg + 4, ...
    const int cl = t & 63, pg = t >> 6;
    for (int sub = c0; sub < c1; sub += 64) {
        const int col = sub + cl;
        // 64 divides HD on the MFMA path; the generic path has one head per segment.
        const int g = sub / HD;
        const int d = min(col, c1 - 1) - g * HD;
        auto row_of = [&](int i) -> int64_t {
            return partial_row(r0 + i, i == 0 && first_tail, p.Hseg, grp) * NH + g;
        };
        float Mt = -INFINITY, Lt = 0.0f, At = 0.0f;  // this thread's partials
        for (int base = pg; base < n; base += 32) {
            float a[8], m[8], l[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {  // unconditional loads (clamped), masked below
                const int64_t row = row_of(min(base + 4 * k, n - 1));
                a[k] = p.ws_acc[row * HD + d];
                m[k] = p.ws_ml[row * 2];
                l[k] = p.ws_ml[row * 2 + 1];
            }
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (base + 4 * k >= n) m[k] = -INFINITY;
            float mb = Mt;
#pragma unroll
            for (int k = 0; k < 8; ++k) mb = fmaxf(mb, m[k]);
            if (mb != -INFINITY) {
                const float sc = fast_exp2(Mt - mb);  // 0 while Mt = -inf
                Lt *= sc;
                At *= sc;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float w = fast_exp2(m[k] - mb);
                    Lt = fmaf(w, l[k], Lt);
                    At = fmaf(w, a[k], At);
                }
                Mt = mb;
            }
        }
        __syncthreads();  // the previous sub-pass has read gm, gl, ga
        if (cl == 0) {
            gm[pg] = Mt;
            gl[pg] = Lt;
        }
        ga[pg][cl] = At;
        __syncthreads();
        if (pg == 0 && col < c1) {
            const float M = fmaxf(fmaxf(gm[0], gm[1]), fmaxf(gm[2], gm[3]));
            float L = 0.0f, A = 0.0f;
            if (M != -INFINITY) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float w = fast_exp2(gm[q] - M);
                    L = fmaf(w, gl[q], L);
                    A = fmaf(w, ga[q][cl], A);
                }
            }
            out0[col] = L > 0.0f ? A / L : 0.0f;
        }
    }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct WorkspaceLayout {
    size_t plan_off, ml_off, acc_off, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Partial slots: 2 per (range, head group), for at most `slots` (range, head
// group) pairs (ranges * Hseg <= slots), each holding NH heads (NH = G for the
// MFMA kernel, 1 for the generic one).  The public size query assumes the
// largest persistent grid (kMaxWaves pairs).
WorkspaceLayout workspace_layout(int B, int Hq, int Hkv, int HD, int slots = kMaxWaves) {
    WorkspaceLayout w{};
    const int G = Hq / std::max(Hkv, 1);
    const size_t head_slots = 2 * static_cast<size_t>(slots) * std::max(G, 1);
    const size_t plan_ints = 5 + static_cast<size_t>(std::min(B, kMaxBatchPerLaunch)) + 1;
    w.plan_off = 0;
    w.ml_off = align256(sizeof(int32_t) * plan_ints);
    w.acc_off = w.ml_off + align256(sizeof(float) * 2 * head_slots);
    w.total = w.acc_off + align256(sizeof(float) * head_slots * HD);
    return w;
}

// Wavefronts of `kernel` resident on the device at once, in workgroups of
// `wpw` wavefronts with `lds` bytes of dynamic LDS each, at most
// `max_per_simd` per SIMD (0 = no cap); cached per device, kernel and LDS size.
template <typename K>
int resident_waves(K kernel, int wpw, size_t lds, int max_per_simd) {
    static std::mutex mu;
    static std::unordered_map<std::string, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    char key[96];
    std::snprintf(key, sizeof(key), "%d:%p:%zu", dev, reinterpret_cast<const void*>(kernel), lds);
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 64 * wpw, lds) != hipSuccess ||
        per_cu <= 0)
        per_cu = std::max(1, 4 / wpw);
    int waves = std::min(kMaxWaves, cus * per_cu * wpw);
    if (max_per_simd > 0) waves = std::min(waves, std::max(wpw, cus * 4 * max_per_simd));
    cache.emplace(key, waves);
    return waves;
}

// Whether a grid of `ranges` ranges is paired (see WorkSplit): the full
// persistent grid at two wavefronts per SIMD, i.e. two workgroups on every
// CU, with an even number of ranges so that the second half of the ranges is
// the second half of the workgroups.
bool paired_grid(const DecodeParams& p, int waves, int max_per_simd) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return false;
    return max_per_simd == 2 && waves == cus * 4 * max_per_simd && p.ranges * p.Hseg == waves && p.ranges % 2 == 0;
}

// Block ranges of the persistent grid: as many as `waves` resident wavefronts
// hold (Hseg per range), no more than the largest possible work needs (small
// batches and short contexts launch a small grid) and no more than the
// workspace has partial slots for.
int decode_ranges(const DecodeParams& p, int waves) {
    const int64_t max_work = static_cast<int64_t>(p.B) * (p.max_blocks + p.seg_cost);
    return static_cast<int>(std::max<int64_t>(
        1, std::min<int64_t>({waves / p.Hseg, cdiv<int64_t>(max_work, p.min_per), p.max_slots / p.Hseg})));
}

// Attention kernel over `ranges * Hseg` persistent wavefronts (workgroups of
// `wpw` of them, wpw dividing Hseg), then the merge.
template <typename K>
int launch_pair(K kern, int wpw, int max_per_simd, DecodeParams p, hipStream_t s, const char* name) {
    const size_t lds = sizeof(int) * (static_cast<size_t>(p.B) + 1);  // the block prefix
    const int waves = resident_waves(kern, wpw, lds, max_per_simd);
    p.ranges = decode_ranges(p, waves);
    p.paired = paired_grid(p, waves, max_per_simd) ? 1 : 0;
    const unsigned groups = static_cast<unsigned>(p.ranges) * (p.Hseg / wpw);
    kern<<<groups, 64 * wpw, lds, s>>>(p);
    if (int rc = check_launch(name)) return rc;
    if (p.ranges == 1) return SKV_OK;  // one range: no segment is cut, nothing to merge
    // Merge grid: about 1,024 workgroups.  Many segments -> one workgroup per
    // segment; few (one long sequence) -> each segment split into 64-column
    // slices merged side by side.
    const int segs = p.B * p.Hseg;
    const int c64 = cdiv(p.NH * p.HD, 64);
    const int split = std::max(1, std::min(c64, 1024 / std::max(segs, 1)));
    p.merge_cw = 64 * cdiv(c64, split);
    const unsigned merge_groups = static_cast<unsigned>(segs) * cdiv(p.NH * p.HD, p.merge_cw);
    decode_merge_kernel<<<merge_groups, 256, 0, s>>>(p);
    return check_launch("decode_merge_kernel");
}

// Wavefronts per workgroup of the MFMA kernel: neighbouring kv heads of the
// same blocks read side by side from one CU (adjacent 256-byte row slices)
// stream faster than when their wavefronts are spread over CUs.
// Launch shape of the MFMA kernel, chosen by measurement on MI355X:
// * 4 wavefronts per workgroup (when Hkv allows): neighbouring kv heads of
//   the same blocks are read side by side from one CU, adjacent 256-byte
//   slices of each row, which streams ~5 % faster than spreading them;
// * a ring of NBUF blocks in flight per wavefront and few wavefronts per
//   SIMD: about 16-24 KiB of K/V requested per SIMD (head_dim 128: 2 blocks
//   of 8 KiB, 1 wavefront per SIMD; head_dim 64: 3 blocks of 4 KiB, 2 per
//   SIMD).  More requests in flight than that lowers the achieved rate.
template <int HD, int G, bool QF32>
int launch_mfma_shape(DecodeParams p, hipStream_t s) {
    constexpr int NB = HD == 64 ? 3 : 2;
    constexpr int PER_SIMD = mfma_waves_per_simd(HD, G);
    const char* name = "decode_mfma_kernel";
    if (p.max_blocks <= 8 * 2) {
        // Short tables (cfg1-like decoding, up to 256 tokens): one workgroup
        // per (sequence, kv head), its 8 wavefronts taking two blocks each,
        // merged in LDS.  Measured at cfg1 (9 blocks): 6.4 us per call, against
        // 7.35 with 4 wavefronts of up to 3 blocks and 6.7 with 12 of one.
        const size_t lds = sizeof(int) * (static_cast<size_t>(p.B) + 1);
        const unsigned groups = static_cast<unsigned>(p.B) * static_cast<unsigned>(p.Hkv);
        decode_mfma_kernel<HD, G, QF32, 8, 2, true><<<groups, 512, lds, s>>>(p);
        return check_launch(name);
    }
    p.seg_cost = kSegmentCost;
    if (p.Hkv % 4 == 0) return launch_pair(decode_mfma_kernel<HD, G, QF32, 4, NB>, 4, PER_SIMD, p, s, name);
    if (p.Hkv % 2 == 0) return launch_pair(decode_mfma_kernel<HD, G, QF32, 2, NB>, 2, PER_SIMD, p, s, name);
    return launch_pair(decode_mfma_kernel<HD, G, QF32, 1, NB>, 1, PER_SIMD, p, s, name);
}

template <bool QF32>
int launch_mfma(const DecodeParams& p, hipStream_t s) {
    const int G = p.Hq / p.Hkv;
#define SKV_MFMA(HD_, G_) \
    if (p.HD == HD_ && G == G_) return launch_mfma_shape<HD_, G_, QF32>(p, s);
    SKV_MFMA(64, 1) SKV_MFMA(64, 2) SKV_MFMA(64, 4) SKV_MFMA(64, 8) SKV_MFMA(64, 16)
    SKV_MFMA(128, 1) SKV_MFMA(128, 2) SKV_MFMA(128, 4) SKV_MFMA(128, 8) SKV_MFMA(128, 16)
#undef SKV_MFMA
    return set_error(SKV_ERR_UNSUPPORTED, "no MFMA decode kernel for head_dim %d, group %d", p.HD, G);
}

// The load-pattern calibration on the grid the MFMA decode kernel (bf16
// queries, stream-K mode) would be launched with for the same geometry.
template <int HD, int G>
int launch_checksum_shape(DecodeParams p, uint32_t* sums, hipStream_t s) {
    constexpr int NB = HD == 64 ? 3 : 2;
    constexpr int PER_SIMD = mfma_waves_per_simd(HD, G);
    const size_t lds = sizeof(int) * (static_cast<size_t>(p.B) + 1);
    p.seg_cost = kSegmentCost;
    auto go = [&](auto decode_kern, auto sum_kern, int wpw) {
        const int waves = resident_waves(decode_kern, wpw, lds, PER_SIMD);
        p.ranges = decode_ranges(p, waves);
        p.paired = paired_grid(p, waves, PER_SIMD) ? 1 : 0;
        const unsigned groups = static_cast<unsigned>(p.ranges) * (p.Hseg / wpw);
        sum_kern<<<groups, 64 * wpw, lds, s>>>(p, sums);
        return check_launch("block_stream_checksum_kernel");
    };
    if (p.Hkv % 4 == 0)
        return go(decode_mfma_kernel<HD, G, false, 4, NB>, block_stream_checksum_kernel<HD, 4, NB>, 4);
    if (p.Hkv % 2 == 0)
        return go(decode_mfma_kernel<HD, G, false, 2, NB>, block_stream_checksum_kernel<HD, 2, NB>, 2);
    return go(decode_mfma_kernel<HD, G, false, 1, NB>, block_stream_checksum_kernel<HD, 1, NB>, 1);
}

int launch_checksum(const DecodeParams& p, uint32_t* sums, hipStream_t s) {
    const int G = p.Hq / p.Hkv;
#define SKV_SUM(HD_, G_) \
    if (p.HD == HD_ && G == G_) return launch_checksum_shape<HD_, G_>(p, sums, s);
    SKV_SUM(64, 1) SKV_SUM(64, 2) SKV_SUM(64, 4) SKV_SUM(64, 8) SKV_SUM(64, 16)
    SKV_SUM(128, 1) SKV_SUM(128, 2) SKV_SUM(128, 4) SKV_SUM(128, 8) SKV_SUM(128, 16)
#undef SKV_SUM
    return set_error(SKV_ERR_UNSUPPORTED, "skv_paged_block_checksum: head_dim %d, group %d has no MFMA decode shape",
                     p.HD, G);
}

bool mfma_path_ok(const DecodeParams& p, int q_dtype) {
    const int G = p.Hq / p.Hkv;
    return p.bs == 16 && (p.HD == 64 || p.HD == 128) &&
           (G == 1 || G == 2 || G == 4 || G == 8 || G == 16) && aligned16(p.k) && aligned16(p.v) &&
           aligned16(p.q) && aligned16(p.out) &&
           (q_dtype == SKV_DTYPE_BF16 || q_dtype == SKV_DTYPE_FP32);
}

// The appended rows go through the MFMA kernel when it runs and its 16-byte
// accesses to them are aligned; otherwise the append kernel runs first (same
// result: it writes position lens[b] - 1 of every sequence, then the decode
// reads it from the pool).
int append_before_decode(DecodeParams& p, hipStream_t s) {
    AppendParams a{p.k_new, p.v_new, p.k_pool_w, p.v_pool_w, p.total_blocks, p.tables,
                   p.max_blocks, p.lens, -1, p.single_len - 1, nullptr, p.B, 1, p.Hkv * p.HD, p.bs};
    p.k_new = p.v_new = nullptr;
    return launch_append(a, p.kv_new_fp32 ? SKV_DTYPE_FP32 : SKV_DTYPE_BF16, s);
}

int run_decode_chunk(DecodeParams p, int q_dtype, char* ws, const WorkspaceLayout& w, hipStream_t s) {
    p.plan = reinterpret_cast<int32_t*>(ws + w.plan_off);
    p.ws_ml = reinterpret_cast<float*>(ws + w.ml_off);
    p.ws_acc = reinterpret_cast<float*>(ws + w.acc_off);
    const bool mfma = mfma_path_ok(p, q_dtype);
    if (p.k_new != nullptr && !(mfma && aligned16(p.k_new) && aligned16(p.v_new)))
        if (int rc = append_before_decode(p, s)) return rc;
    if (mfma) {
        p.Hseg = p.Hkv;
        p.NH = p.Hq / p.Hkv;
        p.min_per = 4;
        return q_dtype == SKV_DTYPE_FP32 ? launch_mfma<true>(p, s) : launch_mfma<false>(p, s);
    }
    p.Hseg = p.Hq;
    p.NH = 1;
    p.min_per = std::max(1, cdiv(64, p.bs));
    return q_dtype == SKV_DTYPE_FP32 ? launch_pair(decode_generic_kernel<true>, 1, 0, p, s, "decode_generic_kernel")
                                     : launch_pair(decode_generic_kernel<false>, 1, 0, p, s, "decode_generic_kernel");
}

// Batches larger than kMaxBatchPerLaunch run as consecutive launches on the
// same stream (sequences are independent), reusing the workspace.
int run_decode(DecodeParams p, int q_dtype, void* workspace, size_t workspace_bytes,
               hipStream_t s, int slots = kMaxWaves) {
    const WorkspaceLayout w = workspace_layout(p.B, p.Hq, p.Hkv, p.HD, slots);
    p.max_slots = slots;
    if (workspace == nullptr || workspace_bytes < w.total)
        return set_error(SKV_ERR_WORKSPACE,
                         "decode workspace of %zu bytes is smaller than the %zu required",
                         workspace_bytes, w.total);
    // Flattened (sequence, block) indices are int32 on the device.
    const long long flat_bound =
        static_cast<long long>(std::min(p.B, kMaxBatchPerLaunch)) * (static_cast<long long>(p.max_blocks) + kSegmentCost);
    if (flat_bound >= (1ll << 30))
        return set_error(SKV_ERR_UNSUPPORTED,
                         "batch x (table width + %d) = %lld exceeds the 2^30 work index range", kSegmentCost,
                         flat_bound);
    const size_t q_elem = q_dtype == SKV_DTYPE_FP32 ? 4 : 2;
    const int B = p.B;
    for (int b0 = 0; b0 < B; b0 += kMaxBatchPerLaunch) {
        DecodeParams c = p;
        c.B = std::min(kMaxBatchPerLaunch, B - b0);
        const size_t head_rows = static_cast<size_t>(b0) * p.Hq * p.HD;
        c.q = static_cast<const char*>(p.q) + head_rows * q_elem;
        c.out = p.out + head_rows;
        c.tables = p.tables + static_cast<int64_t>(b0) * p.max_blocks;
        if (p.lens != nullptr) c.lens = p.lens + b0;
        if (p.k_new != nullptr) {
            const size_t rows = static_cast<size_t>(b0) * p.Hkv * p.HD * (p.kv_new_fp32 ? 4 : 2);
            c.k_new = static_cast<const char*>(p.k_new) + rows;
            c.v_new = static_cast<const char*>(p.v_new) + rows;
        }
        if (int rc = run_decode_chunk(c, q_dtype, static_cast<char*>(workspace), w, s)) return rc;
    }
    return SKV_OK;
}

int validate_geometry(const char* fn, int B, int Hq, int Hkv, int HD, int bs, float scale) {
    SKV_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && HD > 0 && bs > 0,
                "%s: invalid device pointers or attention dimensions", fn);
    SKV_REQUIRE(Hq % Hkv == 0, "%s: num_q_heads %d is not a multiple of num_kv_heads %d", fn, Hq,
                Hkv);
    SKV_REQUIRE(scale > 0.0f && std::isfinite(scale), "%s: scale must be positive and finite", fn);
    if (HD > kMaxHeadDim)
        return set_error(SKV_ERR_UNSUPPORTED, "%s: head_dim %d exceeds %d", fn, HD, kMaxHeadDim);
    return SKV_OK;
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free entry point (skv_paged_decode_append_noalloc):
// the partial results live in this file-scope device array instead of a
// caller workspace.  Each device holds its own copy from module load until the
// process ends.  In host code `scratch` names a host-side stand-in, never a
// device address: its device address comes from hipGetSymbolAddress, once per
// device with that device current, and only that pointer is passed on.
// Nothing in it must start at zero (every partial and the plan are written by
// the attention kernel before the merge kernel reads them).
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = size_t(24) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

int scratch_for_current_device(void** ptr) {
    int dev = 0;
    SKV_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxScratchDevices)
        return set_error(SKV_ERR_UNSUPPORTED, "skv_paged_decode_append_noalloc: device %d beyond %d", dev,
                         kMaxScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* addr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || addr == nullptr)
            return set_error(SKV_ERR_HIP, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = addr;
    }
    *ptr = g_scratch_ptr[dev];
    return SKV_OK;
}

// (range, head group) pairs whose partials fit in the scratch for this shape.
int scratch_slots(int B, int Hq, int Hkv, int HD) {
    int slots = kMaxWaves;
    while (slots > 0 && workspace_layout(B, Hq, Hkv, HD, slots).total > kScratchBytes) slots -= 64;
    return slots;
}

int fill_decode_append(DecodeParams& p, const char* fn, const void* q, int q_dtype, const void* k_new,
                       const void* v_new, int kv_dtype, uint16_t* k_pool, uint16_t* v_pool,
                       int64_t total_blocks, const int32_t* block_tables, int max_blocks_per_seq,
                       const int32_t* context_lens, int num_seqs, int num_q_heads, int num_kv_heads,
                       int head_dim, int block_size, float scale, float* out) {
    SKV_REQUIRE(q && k_new && v_new && k_pool && v_pool && block_tables && context_lens && out,
                "%s: invalid device pointers or attention dimensions", fn);
    SKV_REQUIRE(q_dtype == SKV_DTYPE_BF16 || q_dtype == SKV_DTYPE_FP32, "%s: unknown query dtype %d", fn,
                q_dtype);
    SKV_REQUIRE(kv_dtype == SKV_DTYPE_BF16 || kv_dtype == SKV_DTYPE_FP32, "%s: unknown K/V dtype %d", fn,
                kv_dtype);
    SKV_REQUIRE(total_blocks > 0 && max_blocks_per_seq > 0, "%s: pool and table sizes must be positive", fn);
    if (int rc = validate_geometry(fn, num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, scale))
        return rc;
    p = DecodeParams{};
    p.q = q;
    p.k = k_pool;
    p.v = v_pool;
    p.total_blocks = total_blocks;
    p.tables = block_tables;
    p.max_blocks = max_blocks_per_seq;
    p.lens = context_lens;
    p.single_len = 0;
    p.B = num_seqs;
    p.Hq = num_q_heads;
    p.Hkv = num_kv_heads;
    p.HD = head_dim;
    p.bs = block_size;
    p.qscale = scale * 1.4426950408889634f;
    p.out = out;
    p.k_new = k_new;
    p.v_new = v_new;
    p.kv_new_fp32 = kv_dtype == SKV_DTYPE_FP32 ? 1 : 0;
    p.k_pool_w = k_pool;
    p.v_pool_w = v_pool;
    return SKV_OK;
}

}  // namespace skv

using namespace skv;

extern "C" size_t skv_paged_decode_workspace_bytes(int num_seqs, int num_q_heads, int num_kv_heads,
                                                   int head_dim) {
    if (num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0) return 0;
    return workspace_layout(num_seqs, num_q_heads, num_kv_heads, head_dim).total;
}

extern "C" int skv_paged_decode(const void* q, int q_dtype, const uint16_t* k_pool,
                                const uint16_t* v_pool, int64_t total_blocks,
                                const int32_t* block_tables, int max_blocks_per_seq,
                                const int32_t* context_lens, int num_seqs, int num_q_heads,
                                int num_kv_heads, int head_dim, int block_size, float scale,
                                float* out, void* workspace, size_t workspace_bytes,
                                void* stream) {
    SKV_REQUIRE(q && k_pool && v_pool && block_tables && context_lens && out,
                "skv_paged_decode: invalid device pointers or attention dimensions");
    SKV_REQUIRE(q_dtype == SKV_DTYPE_BF16 || q_dtype == SKV_DTYPE_FP32,
                "skv_paged_decode: unknown query dtype %d", q_dtype);
    SKV_REQUIRE(total_blocks > 0 && max_blocks_per_seq > 0,
                "skv_paged_decode: pool and table sizes must be positive");
    if (int rc = validate_geometry("skv_paged_decode", num_seqs, num_q_heads, num_kv_heads,
                                   head_dim, block_size, scale))
        return rc;
    DecodeParams p{};
    p.q = q;
    p.k = k_pool;
    p.v = v_pool;
    p.total_blocks = total_blocks;
    p.tables = block_tables;
    p.max_blocks = max_blocks_per_seq;
    p.lens = context_lens;
    p.single_len = 0;
    p.B = num_seqs;
    p.Hq = num_q_heads;
    p.Hkv = num_kv_heads;
    p.HD = head_dim;
    p.bs = block_size;
    p.qscale = scale * 1.4426950408889634f;
    p.out = out;
    return run_decode(p, q_dtype, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int skv_paged_decode_append(const void* q, int q_dtype, const void* k_new,
                                       const void* v_new, int kv_dtype, uint16_t* k_pool,
                                       uint16_t* v_pool, int64_t total_blocks,
                                       const int32_t* block_tables, int max_blocks_per_seq,
                                       const int32_t* context_lens, int num_seqs, int num_q_heads,
                                       int num_kv_heads, int head_dim, int block_size, float scale,
                                       float* out, void* workspace, size_t workspace_bytes,
                                       void* stream) {
    DecodeParams p;
    if (int rc = fill_decode_append(p, "skv_paged_decode_append", q, q_dtype, k_new, v_new, kv_dtype, k_pool,
                                    v_pool, total_blocks, block_tables, max_blocks_per_seq, context_lens,
                                    num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, scale, out))
        return rc;
    return run_decode(p, q_dtype, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int skv_paged_decode_append_noalloc(const void* q, int q_dtype, const void* k_new,
                                               const void* v_new, int kv_dtype, uint16_t* k_pool,
                                               uint16_t* v_pool, int64_t total_blocks,
                                               const int32_t* block_tables, int max_blocks_per_seq,
                                               const int32_t* context_lens, int num_seqs,
                                               int num_q_heads, int num_kv_heads, int head_dim,
                                               int block_size, float scale, float* out, void* stream) {
    DecodeParams p;
    if (int rc = fill_decode_append(p, "skv_paged_decode_append_noalloc", q, q_dtype, k_new, v_new, kv_dtype,
                                    k_pool, v_pool, total_blocks, block_tables, max_blocks_per_seq,
                                    context_lens, num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                                    scale, out))
        return rc;
    // At least one range per head group (kv heads for the MFMA kernel, query
    // heads for the generic one) must fit; more ranges are used up to the
    // persistent grid as the scratch allows.
    const int slots = scratch_slots(num_seqs, num_q_heads, num_kv_heads, head_dim);
    if (slots < num_q_heads)
        return set_error(SKV_ERR_UNSUPPORTED,
                         "skv_paged_decode_append_noalloc: %d query heads x head_dim %d need more than the "
                         "%zu-byte scratch", num_q_heads, head_dim, kScratchBytes);
    void* ws = nullptr;
    if (int rc = scratch_for_current_device(&ws)) return rc;
    return run_decode(p, q_dtype, ws, kScratchBytes, static_cast<hipStream_t>(stream), slots);
}

extern "C" size_t skv_paged_attention_decode_workspace_bytes(int num_q_heads, int num_kv_heads,
                                                             int head_dim) {
    return skv_paged_decode_workspace_bytes(1, num_q_heads, num_kv_heads, head_dim);
}

extern "C" int skv_paged_attention_decode(const float* query, const uint16_t* key_cache,
                                          const uint16_t* value_cache, int64_t total_blocks,
                                          const int32_t* block_table, float* output,
                                          int context_len, int block_size, int num_q_heads,
                                          int num_kv_heads, int head_dim, float scale,
                                          void* workspace, size_t workspace_bytes, void* stream) {
    // Same validation as paged_attention_decode_cuda (src/cuda/gemm_cuda.cu:920-928).
    SKV_REQUIRE(query && key_cache && value_cache && block_table && output && context_len > 0 &&
                    total_blocks > 0,
                "paged_attention_decode: invalid device pointers or attention dimensions");
    if (int rc = validate_geometry("paged_attention_decode", 1, num_q_heads, num_kv_heads,
                                   head_dim, block_size, scale))
        return rc;
    DecodeParams p{};
    p.q = query;
    p.k = key_cache;
    p.v = value_cache;
    p.total_blocks = total_blocks;
    p.tables = block_table;
    p.max_blocks = cdiv(context_len, block_size);
    p.lens = nullptr;
    p.single_len = context_len;
    p.B = 1;
    p.Hq = num_q_heads;
    p.Hkv = num_kv_heads;
    p.HD = head_dim;
    p.bs = block_size;
    p.qscale = scale * 1.4426950408889634f;
    p.out = output;
    return run_decode(p, SKV_DTYPE_FP32, workspace, workspace_bytes,
                      static_cast<hipStream_t>(stream));
}

extern "C" int skv_paged_attention_decode_append(const float* query, const void* key_row,
                                                 const void* value_row, int kv_dtype,
                                                 uint16_t* key_cache, uint16_t* value_cache,
                                                 int64_t total_blocks, const int32_t* block_table,
                                                 float* output, int context_len, int block_size,
                                                 int num_q_heads, int num_kv_heads, int head_dim,
                                                 float scale, void* workspace,
                                                 size_t workspace_bytes, void* stream) {
    SKV_REQUIRE(query && key_row && value_row && key_cache && value_cache && block_table &&
                    output && context_len > 0 && total_blocks > 0,
                "paged_attention_decode_append: invalid device pointers or attention dimensions");
    SKV_REQUIRE(kv_dtype == SKV_DTYPE_BF16 || kv_dtype == SKV_DTYPE_FP32,
                "paged_attention_decode_append: unknown K/V dtype %d", kv_dtype);
    if (int rc = validate_geometry("paged_attention_decode_append", 1, num_q_heads, num_kv_heads,
                                   head_dim, block_size, scale))
        return rc;
    DecodeParams p{};
    p.q = query;
    p.k = key_cache;
    p.v = value_cache;
    p.total_blocks = total_blocks;
    p.tables = block_table;
    p.max_blocks = cdiv(context_len, block_size);
    p.lens = nullptr;
    p.single_len = context_len;
    p.B = 1;
    p.Hq = num_q_heads;
    p.Hkv = num_kv_heads;
    p.HD = head_dim;
    p.bs = block_size;
    p.qscale = scale * 1.4426950408889634f;
    p.out = output;
    p.k_new = key_row;
    p.v_new = value_row;
    p.kv_new_fp32 = kv_dtype == SKV_DTYPE_FP32 ? 1 : 0;
    p.k_pool_w = key_cache;
    p.v_pool_w = value_cache;
    return run_decode(p, SKV_DTYPE_FP32, workspace, workspace_bytes,
                      static_cast<hipStream_t>(stream));
}

extern "C" int skv_paged_block_checksum(const uint16_t* k_pool, const uint16_t* v_pool, int64_t total_blocks,
                                        const int32_t* block_tables, int max_blocks_per_seq,
                                        const int32_t* context_lens, int num_seqs, int num_q_heads,
                                        int num_kv_heads, int head_dim, int block_size, uint32_t* checksums,
                                        void* stream) {
    SKV_REQUIRE(k_pool && v_pool && block_tables && context_lens && checksums,
                "skv_paged_block_checksum: invalid device pointers");
    SKV_REQUIRE(total_blocks > 0 && max_blocks_per_seq > 0,
                "skv_paged_block_checksum: pool and table sizes must be positive");
    if (int rc = validate_geometry("skv_paged_block_checksum", num_seqs, num_q_heads, num_kv_heads, head_dim,
                                   block_size, 1.0f))
        return rc;
    DecodeParams p{};
    p.k = k_pool;
    p.v = v_pool;
    p.total_blocks = total_blocks;
    p.tables = block_tables;
    p.max_blocks = max_blocks_per_seq;
    p.lens = context_lens;
    p.B = num_seqs;
    p.Hq = num_q_heads;
    p.Hkv = num_kv_heads;
    p.HD = head_dim;
    p.bs = block_size;
    p.Hseg = num_kv_heads;
    p.NH = num_q_heads / num_kv_heads;
    p.min_per = 4;
    p.max_slots = kMaxWaves;
    if (!mfma_path_ok(p, SKV_DTYPE_BF16) || !aligned16(k_pool) || !aligned16(v_pool))
        return set_error(SKV_ERR_UNSUPPORTED,
                         "skv_paged_block_checksum: needs the MFMA decode geometry (block_size 16, head_dim "
                         "64 or 128, group 1-16, 16-byte aligned pools)");
    if (num_seqs > kMaxBatchPerLaunch ||
        static_cast<long long>(num_seqs) * max_blocks_per_seq >= (1ll << 30))
        return set_error(SKV_ERR_UNSUPPORTED, "skv_paged_block_checksum: at most %d sequences of under 2^30 blocks",
                         kMaxBatchPerLaunch);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    SKV_HIP_TRY(hipMemsetAsync(checksums, 0, sizeof(uint32_t) * static_cast<size_t>(num_seqs) * num_kv_heads, s));
    return launch_checksum(p, checksums, s);
}
