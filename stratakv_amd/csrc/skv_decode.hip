// skv_decode.hip -- paged decode attention (one query token per sequence,
// grouped-query attention over bf16 K/V pools in 16-token blocks).
//
// Replaces paged_attention_decode_kernel / paged_attention_decode_cuda of the
// reference (src/cuda/gemm_cuda.cu:304-429, 915-935).  The reference runs one
// 256-thread block per query head over one sequence, so each K/V byte is read
// by all G = Hq/Hkv query heads of its group, and accumulates P.V in global
// memory.  Here:
//   * work unit = (sequence, kv head, partition of blocks).  One wavefront owns
//     a unit and serves all G query heads of the group from one read of K/V.
//   * a device-side planner sizes partitions from the actual context lengths
//     so the grid holds ~16k units whatever the batch / length mix ("split-K",
//     the flash-decoding scheme), and a merge kernel combines the partial
//     (max, sum, acc) triples of sequences that span several partitions with
//     a log-sum-exp rescale.
//   * a block's rows are read 16 bytes per lane: HD/8 lanes cover one 128 or
//     256-byte row, so one load instruction moves 64/(HD/8) full rows.
//   * q.k partial dots are reduced across the lanes of a row with DPP
//     butterflies (no LDS); every row group keeps its own online-softmax state
//     and the groups are merged once per unit.
// Softmax runs in the exp2 domain: q is pre-multiplied by scale*log2(e).
#include "skv_common.h"

#include <algorithm>
#include <cmath>

namespace skv {

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
    int32_t* plan;         // [B + 2]: part_base[0..B], blocks per unit at [B + 1]
    float* ws_ml;          // [parts_cap][Hq][2]  (running max in log2 units, sum)
    float* ws_acc;         // [parts_cap][Hq][HD] (unnormalised P.V)
    int target_parts;
    int min_bpu;
};

constexpr int kTargetUnits = 16384;  // ~64 wavefronts of work per CU
constexpr int kMaxHeadDim = 512;

__host__ __device__ inline int parts_target(int Hkv) {
    return std::max(1, kTargetUnits / Hkv);
}

__device__ __forceinline__ int seq_len(const DecodeParams& p, int b) {
    return p.lens != nullptr ? p.lens[b] : p.single_len;
}

__device__ __forceinline__ int seq_blocks(const DecodeParams& p, int b) {
    const int L = seq_len(p, b);
    if (L <= 0) return 0;
    return std::min(cdiv(L, p.bs), p.max_blocks);
}

// ---------------------------------------------------------------------------
// Planner: one workgroup.  blocks per unit = max(min_bpu, ceil(sum_b nb_b /
// target_parts)); parts_b = ceil(nb_b / bpu); part_base = exclusive scan.
// Since parts_b <= nb_b/bpu + 1, the total is at most target_parts + B.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void decode_plan_kernel(DecodeParams p) {
    __shared__ long long s_red[1024];
    __shared__ int s_scan[1024];
    const int t = threadIdx.x, nt = blockDim.x;
    const int per = cdiv(p.B, nt);
    const int b0 = std::min(t * per, p.B), b1 = std::min(b0 + per, p.B);

    long long mine = 0;
    for (int b = b0; b < b1; ++b) mine += seq_blocks(p, b);
    s_red[t] = mine;
    __syncthreads();
    for (int o = nt / 2; o > 0; o >>= 1) {
        if (t < o) s_red[t] += s_red[t + o];
        __syncthreads();
    }
    const long long total_blocks = s_red[0];
    const int bpu = static_cast<int>(
        std::max<long long>(p.min_bpu, cdiv<long long>(total_blocks, p.target_parts)));

    int parts = 0;
    for (int b = b0; b < b1; ++b) parts += cdiv(seq_blocks(p, b), bpu);
    s_scan[t] = parts;
    __syncthreads();
    for (int o = 1; o < nt; o <<= 1) {  // inclusive Hillis-Steele scan
        const int add = t >= o ? s_scan[t - o] : 0;
        __syncthreads();
        s_scan[t] += add;
        __syncthreads();
    }
    int base = s_scan[t] - parts;
    for (int b = b0; b < b1; ++b) {
        p.plan[b] = base;
        base += cdiv(seq_blocks(p, b), bpu);
    }
    if (t == nt - 1) {
        p.plan[p.B] = s_scan[t];
        p.plan[p.B + 1] = bpu;
    }
}

// Locate the sequence owning global partition pg: part_base[b] <= pg < part_base[b+1].
__device__ __forceinline__ int find_seq(const int32_t* plan, int B, int pg) {
    int lo = 0, hi = B;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (plan[mid] <= pg) lo = mid; else hi = mid;
    }
    return lo;
}

// ---------------------------------------------------------------------------
// Fast path: block_size 16, head_dim 64 or 128, G in {1,2,4,8}.
// Lane layout: LPR = HD/8 lanes per K/V row (8 elements = 16 bytes each),
// RPI = 64/LPR rows per load instruction, TPL = 16/RPI rows per lane per block.
// Lane (r, c) handles rows r, r+RPI, ... of every block, elements [8c, 8c+8).
// ---------------------------------------------------------------------------
template <int HD, int G, bool QF32>
__global__ __launch_bounds__(64) void decode_fast_kernel(DecodeParams p) {
    constexpr int BS = 16;
    constexpr int LPR = HD / 8;
    constexpr int RPI = 64 / LPR;
    constexpr int TPL = BS / RPI;
    static_assert(LPR * RPI == 64 && RPI * TPL == BS, "lane layout");

    const int lane = threadIdx.x;
    const int r = lane / LPR, c = lane % LPR;
    const int Hkv = p.Hkv;
    const int total_parts = p.plan[p.B];
    const int u = blockIdx.x;
    if (u >= total_parts * Hkv) return;
    const int pg = u / Hkv;
    const int kvh = u - pg * Hkv;
    const int b = find_seq(p.plan, p.B, pg);
    const int part = pg - p.plan[b];
    const int nparts = p.plan[b + 1] - p.plan[b];
    const int bpu = p.plan[p.B + 1];
    const int L = seq_len(p, b);
    const int nb = std::min(cdiv(L, BS), p.max_blocks);
    const int Leff = std::min(L, nb * BS);
    const int blk0 = part * bpu;
    const int blk1 = std::min(blk0 + bpu, nb);
    const int32_t* table = p.tables + static_cast<int64_t>(b) * p.max_blocks;
    const int h0 = kvh * G;

    float qf[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int64_t qoff = (static_cast<int64_t>(b) * p.Hq + h0 + g) * HD + 8 * c;
        if constexpr (QF32) {
            const float4* qp = reinterpret_cast<const float4*>(static_cast<const float*>(p.q) + qoff);
            const float4 a0 = qp[0], a1 = qp[1];
            qf[g][0] = a0.x; qf[g][1] = a0.y; qf[g][2] = a0.z; qf[g][3] = a0.w;
            qf[g][4] = a1.x; qf[g][5] = a1.y; qf[g][6] = a1.z; qf[g][7] = a1.w;
        } else {
            const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.q) + qoff);
            unpack8(w, qf[g]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) qf[g][j] *= p.qscale;
    }

    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[g][j] = 0.0f;
    }

    const int64_t row_stride = static_cast<int64_t>(Hkv) * HD;
    const int64_t lane_off = static_cast<int64_t>(kvh) * HD + 8 * c + static_cast<int64_t>(r) * row_stride;

    for (int blk = blk0; blk < blk1; ++blk) {
        const int64_t pb = table[blk];
        if (pb < 0 || pb >= p.total_blocks) continue;
        const uint16_t* kb = p.k + pb * BS * row_stride + lane_off;
        const uint16_t* vb = p.v + pb * BS * row_stride + lane_off;
        uint4 kw[TPL], vw[TPL];
#pragma unroll
        for (int i = 0; i < TPL; ++i) {
            kw[i] = *reinterpret_cast<const uint4*>(kb + static_cast<int64_t>(i) * RPI * row_stride);
            vw[i] = *reinterpret_cast<const uint4*>(vb + static_cast<int64_t>(i) * RPI * row_stride);
        }
        float s[TPL][G];
#pragma unroll
        for (int i = 0; i < TPL; ++i) {
            float kf[8];
            unpack8(kw[i], kf);
            const bool valid = blk * BS + i * RPI + r < Leff;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float d = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) d = fmaf(qf[g][j], kf[j], d);
                d = group_sum<LPR>(d);
                s[i][g] = valid ? d : -INFINITY;
            }
        }
        float vf[TPL][8];
#pragma unroll
        for (int i = 0; i < TPL; ++i) unpack8(vw[i], vf[i]);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float mb = s[0][g];
#pragma unroll
            for (int i = 1; i < TPL; ++i) mb = fmaxf(mb, s[i][g]);
            const float mn = fmaxf(m[g], mb);
            const float ms = mn == -INFINITY ? 0.0f : mn;
            const float alpha = fast_exp2(m[g] - ms);
            m[g] = mn;
            l[g] *= alpha;
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[g][j] *= alpha;
#pragma unroll
            for (int i = 0; i < TPL; ++i) {
                const float pp = fast_exp2(s[i][g] - ms);
                l[g] += pp;
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[g][j] = fmaf(pp, vf[i][j], acc[g][j]);
            }
        }
    }

    // Merge the RPI row groups (lanes c, c+LPR, ...) into every lane.
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mo = shfl_xor_f(m[g], off);
            const float lo = shfl_xor_f(l[g], off);
            const float mn = fmaxf(m[g], mo);
            const float ms = mn == -INFINITY ? 0.0f : mn;
            const float sa = fast_exp2(m[g] - ms);
            const float sb = fast_exp2(mo - ms);
            l[g] = l[g] * sa + lo * sb;
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[g][j] = acc[g][j] * sa + shfl_xor_f(acc[g][j], off) * sb;
            m[g] = mn;
        }
    }

    if (r != 0) return;
    if (nparts == 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float inv = l[g] > 0.0f ? 1.0f / l[g] : 0.0f;
            float4* o = reinterpret_cast<float4*>(
                p.out + (static_cast<int64_t>(b) * p.Hq + h0 + g) * HD + 8 * c);
            o[0] = make_float4(acc[g][0] * inv, acc[g][1] * inv, acc[g][2] * inv, acc[g][3] * inv);
            o[1] = make_float4(acc[g][4] * inv, acc[g][5] * inv, acc[g][6] * inv, acc[g][7] * inv);
        }
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int64_t row = static_cast<int64_t>(pg) * p.Hq + h0 + g;
            float4* o = reinterpret_cast<float4*>(p.ws_acc + row * HD + 8 * c);
            o[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
            o[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
            if (c == 0) {
                p.ws_ml[row * 2 + 0] = m[g];
                p.ws_ml[row * 2 + 1] = l[g];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Generic path: any block size, head_dim <= 512, any group size.  One
// wavefront per (partition, query head): lanes own tokens for q.k (q staged in
// LDS) and head dimensions for P.V.  Correct for every shape the reference
// accepts; the fast path covers the benchmark geometries.
// ---------------------------------------------------------------------------
template <bool QF32>
__global__ __launch_bounds__(64) void decode_generic_kernel(DecodeParams p) {
    constexpr int DPL = kMaxHeadDim / 64;
    __shared__ float q_s[kMaxHeadDim];
    __shared__ float p_s[64];
    __shared__ int64_t row_s[64];

    const int lane = threadIdx.x;
    const int total_parts = p.plan[p.B];
    const int u = blockIdx.x;
    if (u >= total_parts * p.Hq) return;
    const int pg = u / p.Hq;
    const int h = u - pg * p.Hq;
    const int b = find_seq(p.plan, p.B, pg);
    const int part = pg - p.plan[b];
    const int nparts = p.plan[b + 1] - p.plan[b];
    const int bpu = p.plan[p.B + 1];
    const int L = seq_len(p, b);
    const int nb = std::min(cdiv(L, p.bs), p.max_blocks);
    const int Leff = std::min(L, nb * p.bs);
    const int tok0 = part * bpu * p.bs;
    const int tok1 = std::min((part * bpu + bpu) * p.bs, Leff);
    const int kvh = h / (p.Hq / p.Hkv);
    const int HD = p.HD;
    const int32_t* table = p.tables + static_cast<int64_t>(b) * p.max_blocks;

    const int64_t qoff = (static_cast<int64_t>(b) * p.Hq + h) * HD;
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
    const int64_t row_elems = static_cast<int64_t>(p.Hkv) * HD;

    for (int t0 = tok0; t0 < tok1; t0 += 64) {
        const int t = t0 + lane;
        float score = -INFINITY;
        int64_t roff = -1;
        if (t < tok1) {
            const int64_t pb = table[t / p.bs];
            if (pb >= 0 && pb < p.total_blocks) {
                roff = (pb * p.bs + t % p.bs) * row_elems + static_cast<int64_t>(kvh) * HD;
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
        for (int j = 0; j < n; ++j) {
            const int64_t vr = row_s[j];
            if (vr < 0) continue;
            const float pj = p_s[j];
            const uint16_t* vrow = p.v + vr;
#pragma unroll
            for (int k = 0; k < DPL; ++k) {
                const int d = lane + 64 * k;
                if (d < HD) acc[k] = fmaf(pj, bf16_to_f32(vrow[d]), acc[k]);
            }
        }
        __syncthreads();
    }

    if (nparts == 1) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float* o = p.out + (static_cast<int64_t>(b) * p.Hq + h) * HD;
#pragma unroll
        for (int k = 0; k < DPL; ++k) {
            const int d = lane + 64 * k;
            if (d < HD) o[d] = acc[k] * inv;
        }
    } else {
        const int64_t row = static_cast<int64_t>(pg) * p.Hq + h;
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
}

// ---------------------------------------------------------------------------
// Merge: one workgroup per (sequence, query head).  Sequences with a single
// partition were finalised by the attention kernel; sequences without context
// get zeros.  out = sum_p acc_p 2^(m_p - M) / sum_p l_p 2^(m_p - M).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeParams p) {
    constexpr int kChunk = 2048;
    __shared__ float w_s[kChunk];
    __shared__ float red[256];
    const int t = threadIdx.x;
    const int b = blockIdx.x / p.Hq;
    const int h = blockIdx.x - b * p.Hq;
    const int base = p.plan[b];
    const int nparts = p.plan[b + 1] - base;
    if (nparts == 1) return;
    const int HD = p.HD;
    float* o = p.out + (static_cast<int64_t>(b) * p.Hq + h) * HD;
    if (nparts == 0) {
        for (int d = t; d < HD; d += 256) o[d] = 0.0f;
        return;
    }
    auto ml = [&](int i, int which) {
        return p.ws_ml[(static_cast<int64_t>(base + i) * p.Hq + h) * 2 + which];
    };

    float mx = -INFINITY;
    for (int i = t; i < nparts; i += 256) mx = fmaxf(mx, ml(i, 0));
    red[t] = mx;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (t < s) red[t] = fmaxf(red[t], red[t + s]);
        __syncthreads();
    }
    const float M = red[0];
    const float Ms = M == -INFINITY ? 0.0f : M;
    __syncthreads();

    // Threads split into S slices of HD dims; slice s handles parts i = s mod S.
    const int S = HD <= 256 ? 256 / HD : 1;
    const int slice = t / std::min(HD, 256);
    const int d0 = t % std::min(HD, 256);
    float acc[2] = {0.0f, 0.0f};  // HD <= 512: at most two dims per thread
    float lsum = 0.0f;
    for (int c0 = 0; c0 < nparts; c0 += kChunk) {
        const int n = std::min(kChunk, nparts - c0);
        for (int i = t; i < n; i += 256) {
            const float w = fast_exp2(ml(c0 + i, 0) - Ms);
            w_s[i] = w;
            lsum += ml(c0 + i, 1) * w;
        }
        __syncthreads();
        if (slice < S) {
            for (int i = slice; i < n; i += S) {
                const float w = w_s[i];
                const float* a = p.ws_acc + (static_cast<int64_t>(base + c0 + i) * p.Hq + h) * HD;
                acc[0] = fmaf(w, a[d0], acc[0]);
                if (d0 + 256 < HD) acc[1] = fmaf(w, a[d0 + 256], acc[1]);
            }
        }
        __syncthreads();
    }
    red[t] = lsum;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (t < s) red[t] += red[t + s];
        __syncthreads();
    }
    const float total = red[0];
    const float inv = total > 0.0f ? 1.0f / total : 0.0f;
    __syncthreads();
    // Reduce the S slices of the first 256 dims through LDS.
    red[t] = slice < S ? acc[0] : 0.0f;
    __syncthreads();
    if (slice == 0) {
        float sum = red[t];
        for (int s = 1; s < S; ++s) sum += red[t + s * HD];
        if (d0 < HD) o[d0] = sum * inv;
        if (d0 + 256 < HD) o[d0 + 256] = acc[1] * inv;
    }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct WorkspaceLayout {
    size_t plan_off, ml_off, acc_off, total;
    int parts_cap;
};

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

WorkspaceLayout workspace_layout(int B, int Hq, int Hkv, int HD) {
    WorkspaceLayout w{};
    w.parts_cap = parts_target(Hkv) + B;
    w.plan_off = 0;
    w.ml_off = align256(sizeof(int32_t) * (static_cast<size_t>(B) + 2));
    w.acc_off = w.ml_off + align256(sizeof(float) * 2 * static_cast<size_t>(w.parts_cap) * Hq);
    w.total = w.acc_off + align256(sizeof(float) * static_cast<size_t>(w.parts_cap) * Hq * HD);
    return w;
}

template <bool QF32>
int launch_fast(const DecodeParams& p, unsigned grid, hipStream_t s) {
    const int G = p.Hq / p.Hkv;
#define SKV_FAST(HD_, G_)                                                          \
    if (p.HD == HD_ && G == G_) {                                                  \
        decode_fast_kernel<HD_, G_, QF32><<<grid, 64, 0, s>>>(p);                  \
        return check_launch("decode_fast_kernel");                                 \
    }
    SKV_FAST(64, 1) SKV_FAST(64, 2) SKV_FAST(64, 4) SKV_FAST(64, 8)
    SKV_FAST(128, 1) SKV_FAST(128, 2) SKV_FAST(128, 4) SKV_FAST(128, 8)
#undef SKV_FAST
    return set_error(SKV_ERR_UNSUPPORTED, "no fast decode kernel for head_dim %d, group %d", p.HD, G);
}

bool fast_path_ok(const DecodeParams& p, int q_dtype) {
    const int G = p.Hq / p.Hkv;
    return p.bs == 16 && (p.HD == 64 || p.HD == 128) && (G == 1 || G == 2 || G == 4 || G == 8) &&
           aligned16(p.k) && aligned16(p.v) && aligned16(p.q) && aligned16(p.out) &&
           (q_dtype == SKV_DTYPE_BF16 || q_dtype == SKV_DTYPE_FP32);
}

int run_decode(DecodeParams p, int q_dtype, void* workspace, size_t workspace_bytes,
               hipStream_t s) {
    const WorkspaceLayout w = workspace_layout(p.B, p.Hq, p.Hkv, p.HD);
    if (workspace == nullptr || workspace_bytes < w.total)
        return set_error(SKV_ERR_WORKSPACE,
                         "decode workspace of %zu bytes is smaller than the %zu required",
                         workspace_bytes, w.total);
    char* ws = static_cast<char*>(workspace);
    p.plan = reinterpret_cast<int32_t*>(ws + w.plan_off);
    p.ws_ml = reinterpret_cast<float*>(ws + w.ml_off);
    p.ws_acc = reinterpret_cast<float*>(ws + w.acc_off);
    p.target_parts = parts_target(p.Hkv);
    p.min_bpu = std::max(1, cdiv(64, p.bs));

    decode_plan_kernel<<<1, 1024, 0, s>>>(p);
    if (int rc = check_launch("decode_plan_kernel")) return rc;

    int rc;
    if (fast_path_ok(p, q_dtype)) {
        const unsigned grid = static_cast<unsigned>(w.parts_cap) * p.Hkv;
        rc = q_dtype == SKV_DTYPE_FP32 ? launch_fast<true>(p, grid, s) : launch_fast<false>(p, grid, s);
    } else {
        const unsigned grid = static_cast<unsigned>(w.parts_cap) * p.Hq;
        if (q_dtype == SKV_DTYPE_FP32)
            decode_generic_kernel<true><<<grid, 64, 0, s>>>(p);
        else
            decode_generic_kernel<false><<<grid, 64, 0, s>>>(p);
        rc = check_launch("decode_generic_kernel");
    }
    if (rc) return rc;

    decode_merge_kernel<<<static_cast<unsigned>(p.B) * p.Hq, 256, 0, s>>>(p);
    return check_launch("decode_merge_kernel");
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
