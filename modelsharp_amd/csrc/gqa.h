// gqa.h — GroupQueryAttention (com.microsoft), the attention of Llama-family decoder
// layers between the q/k/v and o projections (Cpu/Kernels/Llm/GroupQueryAttentionKernel.cs).
//
//   num_heads query heads share kv_num_heads key/value heads (group = num_heads / kv_heads);
//   causal: query qi (absolute position past + qi) sees keys
//     [max(0, qAbs - local_window_size + 1) if the window is set, else 0,
//      min(qAbs, seqlens_k[b])];
//   optional rotary on Q and K (not V) from cos/sin caches indexed by absolute position
//     (half-split or interleaved pairs, channels past the rotary span unchanged);
//   present K/V = past rows, then the new rows, [B, kv_heads, capacity, head_dim];
//   out = softmax(scale * q.K^T) V with the row maximum subtracted before exp.
//
// Present buffers carry a row capacity: a caller that keeps its cache in HBM passes the
// same buffer as past and present (past_in_present) and each step appends only its new
// rows — the append-only cache the reference's CPU kernel cannot keep (:239-253).
//
// Kernels:
//   gqa_copy_past_kernel  past -> present rows [0, past) (skipped for an in-place cache)
//   gqa_append_kernel     one thread per channel of each new (token, kv head) row: K
//                         rotated exactly as the reference's ApplyRotary (:330-370,
//                         a * c - b * s and b * c + a * s, each product rounded), V copied
//   gqa_rows_kernel<G>    head_dim = 4 G in {32, 64, 128, 256}: one workgroup per (unit,
//                         key split), units in the reference's order (:283-287). G lanes
//                         read one key (value) row as float4s, coalesced; 256 / G rows are
//                         in flight per pass, four passes' loads issued before their math.
//                         q.k is reduced over the G lanes by xor shuffles; the split's
//                         scores sit in LDS; a fixed-order tree gives the maximum and the
//                         sum; the weighted V rows are summed per lane group and the groups
//                         added in order. One split: the output row. Several (few units,
//                         long history): each writes (max, sum, unnormalised row) and
//   gqa_combine_kernel    rescales the splits to the common maximum and normalises
//   gqa_attention_kernel  any other head_dim: one workgroup per unit, keys strided over
//                         the threads
#pragma once
#include "decoder_ops.h"

namespace msnb {

struct GqaArgs {
    const float* q;       // query rows [B * Sq][q_stride]
    const float* k;       // new key rows [B * Skv][kv_stride] (packed: inside the query rows)
    const float* v;
    const float* past_k;  // [B, kvH, past, D] (unused when past_in_present)
    const float* past_v;
    const int32_t* seqlens;
    const float* cos;     // [cache_rows][half]
    const float* sin;
    float* out;           // [B * Sq][H * D]
    float* pk;            // [B, kvH, cap, D]
    float* pv;
    int B, Sq, Skv, H, kvH, D, past, cap, total;
    int q_stride, kv_stride;
    int seqlens_len;
    int do_rotary, interleaved, half, rot_half, cache_rows;
    int window;
    float scale;
};

__device__ __forceinline__ float rotated(const float* row, int d, int pos, const GqaArgs& p)
{
    const int rot = 2 * p.rot_half;
    if (!p.do_rotary || d >= rot) return row[d];
    int j, i0, i1;
    if (p.interleaved) {
        j = d >> 1;
        i0 = 2 * j;
        i1 = i0 + 1;
    } else {
        j = d < p.rot_half ? d : d - p.rot_half;
        i0 = j;
        i1 = j + p.rot_half;
    }
    const float c = p.cos[(int64_t)pos * p.half + j], s = p.sin[(int64_t)pos * p.half + j];
    const float a = row[i0], b = row[i1];
    return d == i0 ? a * c - b * s : b * c + a * s;
}

__device__ __forceinline__ int rotary_pos(int pos, const GqaArgs& p)
{
    return pos >= p.cache_rows ? p.cache_rows - 1 : pos;
}

__global__ __launch_bounds__(256) void gqa_copy_past_kernel(GqaArgs p)
{
    const int64_t n = (int64_t)p.B * p.kvH * p.past * p.D;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t bg = i / ((int64_t)p.past * p.D);
        const int64_t rem = i - bg * p.past * p.D;
        const int64_t dst = bg * p.cap * p.D + rem;
        p.pk[dst] = p.past_k[i];
        p.pv[dst] = p.past_v[i];
    }
}

// grid: B * Skv * kvH rows, blockDim >= D (one thread per channel)
__global__ __launch_bounds__(256) void gqa_append_kernel(GqaArgs p)
{
    const int row = blockIdx.x;   // (b, s, g) in the reference's scatter order (:255-263)
    const int g = row % p.kvH, bs = row / p.kvH;
    const int s = bs % p.Skv, b = bs / p.Skv;
    const float* krow = p.k + (int64_t)(b * p.Skv + s) * p.kv_stride + g * p.D;
    const float* vrow = p.v + (int64_t)(b * p.Skv + s) * p.kv_stride + g * p.D;
    const int pos = rotary_pos(p.past + s, p);
    const int64_t dst = ((int64_t)(b * p.kvH + g) * p.cap + p.past + s) * p.D;
    for (int d = threadIdx.x; d < p.D; d += blockDim.x) {
        p.pk[dst + d] = rotated(krow, d, pos, p);
        p.pv[dst + d] = vrow[d];
    }
}

constexpr int kGqaThreads = 256;

__device__ __forceinline__ float block_max256(float v, float* red)
{
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return m;
}

// Dynamic LDS: q[D], part[max(256, D)], scores[total]
__global__ __launch_bounds__(kGqaThreads) void gqa_attention_kernel(GqaArgs p)
{
    extern __shared__ float lds[];
    __shared__ float red[4];
    float* qs = lds;
    float* part = lds + p.D;
    float* scores = part + max(kGqaThreads, p.D);
    const int unit = blockIdx.x;
    const int qi = unit % p.Sq, hb = unit / p.Sq;
    const int h = hb % p.H, b = hb / p.H;
    const int g = h / (p.H / p.kvH);
    const int tid = threadIdx.x;

    int bound = p.total - 1;
    if (p.seqlens_len > 0) bound = min(bound, p.seqlens[min(b, p.seqlens_len - 1)]);
    const int q_abs = p.past + qi;
    const int k_limit = min(q_abs, bound);
    const int k_start = p.window >= 0 ? max(0, q_abs - p.window + 1) : 0;
    const int L = k_limit - k_start + 1;

    const float* qrow = p.q + (int64_t)(b * p.Sq + qi) * p.q_stride + h * p.D;
    const int pos = rotary_pos(q_abs, p);
    for (int d = tid; d < p.D; d += kGqaThreads) qs[d] = rotated(qrow, d, pos, p);
    __syncthreads();

    const float* kbase = p.pk + ((int64_t)(b * p.kvH + g) * p.cap + k_start) * p.D;
    const float* vbase = p.pv + ((int64_t)(b * p.kvH + g) * p.cap + k_start) * p.D;
    float* orow = p.out + (int64_t)(b * p.Sq + qi) * p.H * p.D + h * p.D;

    // scores
    float mx = -__builtin_inff();
    for (int j = tid; j < L; j += kGqaThreads) {
        const float* kr = kbase + (int64_t)j * p.D;
        float dot = 0.0f;
        if ((p.D & 3) == 0) {
            for (int d = 0; d < p.D; d += 4) {
                const float4 k4 = *reinterpret_cast<const float4*>(kr + d);
                dot = __builtin_fmaf(qs[d], k4.x, dot);
                dot = __builtin_fmaf(qs[d + 1], k4.y, dot);
                dot = __builtin_fmaf(qs[d + 2], k4.z, dot);
                dot = __builtin_fmaf(qs[d + 3], k4.w, dot);
            }
        } else {
            for (int d = 0; d < p.D; ++d) dot = __builtin_fmaf(qs[d], kr[d], dot);
        }
        const float sc = dot * p.scale;
        scores[j] = sc;
        mx = fmaxf(mx, sc);
    }
    mx = block_max256(mx, red);
    float sum = 0.0f;
    for (int j = tid; j < L; j += kGqaThreads) {
        const float e = expf(scores[j] - mx);
        scores[j] = e;
        sum = sum + e;
    }
    sum = block_sum256(sum, red);   // also orders the score writes before the reads below
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;

    // out[d] = sum_j (e_j * inv) * v[j][d]: chunk c of the keys per thread group
    const int nch = p.D <= kGqaThreads ? kGqaThreads / p.D : 1;
    const int c = tid / p.D;
    if (p.D <= kGqaThreads) {
        const int d = tid - c * p.D;
        if (c < nch) {
            const int j0 = (int)(((int64_t)L * c) / nch), j1 = (int)(((int64_t)L * (c + 1)) / nch);
            float acc = 0.0f;
            for (int j = j0; j < j1; ++j) acc = __builtin_fmaf(scores[j] * inv, vbase[(int64_t)j * p.D + d], acc);
            part[c * p.D + d] = acc;
        }
        __syncthreads();
        if (tid < p.D) {
            float o = part[tid];
            for (int cc = 1; cc < nch; ++cc) o = o + part[cc * p.D + tid];
            orow[tid] = L > 0 ? o : 0.0f;
        }
    } else {
        for (int d = tid; d < p.D; d += kGqaThreads) {
            float acc = 0.0f;
            for (int j = 0; j < L; ++j) acc = __builtin_fmaf(scores[j] * inv, vbase[(int64_t)j * p.D + d], acc);
            orow[d] = acc;
        }
    }
}

constexpr int kGqaMaxSplits = 64;

// Geometry of one (batch, head, query) unit.
struct GqaUnit {
    int b, h, qi, g, k_start, L;
};

__device__ __forceinline__ GqaUnit gqa_unit(const GqaArgs& p, int unit)
{
    GqaUnit u;
    u.qi = unit % p.Sq;
    const int hb = unit / p.Sq;
    u.h = hb % p.H;
    u.b = hb / p.H;
    u.g = u.h / (p.H / p.kvH);
    int bound = p.total - 1;
    if (p.seqlens_len > 0) bound = min(bound, p.seqlens[min(u.b, p.seqlens_len - 1)]);
    const int q_abs = p.past + u.qi;
    const int k_limit = min(q_abs, bound);
    u.k_start = p.window >= 0 ? max(0, q_abs - p.window + 1) : 0;
    u.L = k_limit - u.k_start + 1;
    return u;
}

// Dynamic LDS: q[D], part[(256 / G) * D], scores[ceil(L / splits)]
template <int G>
__global__ __launch_bounds__(kGqaThreads) void gqa_rows_kernel(GqaArgs p, float* __restrict__ ws, int splits)
{
    constexpr int NG = kGqaThreads / G, D = 4 * G, U = 4;
    extern __shared__ float lds[];
    __shared__ float red[4];
    float* qs = lds;
    float* part = qs + D;
    float* scores = part + NG * D;
    const int unit = blockIdx.x / splits, sp = blockIdx.x - unit * splits;
    const GqaUnit u = gqa_unit(p, unit);
    const int L = max(u.L, 0);
    const int j0 = (int)(((int64_t)L * sp) / splits), j1 = (int)(((int64_t)L * (sp + 1)) / splits);
    const int Ls = j1 - j0;
    const int tid = threadIdx.x, kg = tid / G, e = tid - kg * G;

    const float* qrow = p.q + (int64_t)(u.b * p.Sq + u.qi) * p.q_stride + u.h * D;
    const int pos = rotary_pos(p.past + u.qi, p);
    for (int d = tid; d < D; d += kGqaThreads) qs[d] = rotated(qrow, d, pos, p);
    __syncthreads();
    const float4 q4 = *reinterpret_cast<const float4*>(qs + 4 * e);
    const int64_t row0 = ((int64_t)(u.b * p.kvH + u.g) * p.cap + u.k_start + j0) * D + 4 * e;
    const float* kb = p.pk + row0;
    const float* vb = p.pv + row0;

    float mx = -__builtin_inff();
    for (int j = kg; j < Ls; j += U * NG) {
        float4 k4[U];
#pragma unroll
        for (int t = 0; t < U; ++t) {
            const int jj = j + t * NG;
            k4[t] = jj < Ls ? *reinterpret_cast<const float4*>(kb + (int64_t)jj * D) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int t = 0; t < U; ++t) {
            float d = q4.x * k4[t].x;
            d = __builtin_fmaf(q4.y, k4[t].y, d);
            d = __builtin_fmaf(q4.z, k4[t].z, d);
            d = __builtin_fmaf(q4.w, k4[t].w, d);
#pragma unroll
            for (int o = G / 2; o > 0; o >>= 1) d += __shfl_xor(d, o, G);
            const int jj = j + t * NG;
            if (jj < Ls) {
                const float sc = d * p.scale;
                if (e == 0) scores[jj] = sc;
                mx = fmaxf(mx, sc);
            }
        }
    }
    mx = block_max256(mx, red);
    float sum = 0.0f;
    for (int j = tid; j < Ls; j += kGqaThreads) {
        const float ex = expf(scores[j] - mx);
        scores[j] = ex;
        sum = sum + ex;
    }
    sum = block_sum256(sum, red);   // also orders the score writes before the reads below
    const float inv = splits == 1 ? (sum > 0.0f ? 1.0f / sum : 0.0f) : 1.0f;

    float4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = kg; j < Ls; j += U * NG) {
        float4 v4[U];
#pragma unroll
        for (int t = 0; t < U; ++t) {
            const int jj = j + t * NG;
            v4[t] = jj < Ls ? *reinterpret_cast<const float4*>(vb + (int64_t)jj * D) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int t = 0; t < U; ++t) {
            const int jj = j + t * NG;
            if (jj < Ls) {
                const float w = scores[jj] * inv;
                acc.x = __builtin_fmaf(w, v4[t].x, acc.x);
                acc.y = __builtin_fmaf(w, v4[t].y, acc.y);
                acc.z = __builtin_fmaf(w, v4[t].z, acc.z);
                acc.w = __builtin_fmaf(w, v4[t].w, acc.w);
            }
        }
    }
    *reinterpret_cast<float4*>(part + kg * D + 4 * e) = acc;
    __syncthreads();
    for (int d = tid; d < D; d += kGqaThreads) {
        float o = part[d];
        for (int c = 1; c < NG; ++c) o = o + part[c * D + d];
        if (splits == 1) {
            p.out[(int64_t)(u.b * p.Sq + u.qi) * p.H * D + u.h * D + d] = L > 0 ? o : 0.0f;
        } else {
            ws[(int64_t)blockIdx.x * (D + 2) + d] = o;
        }
    }
    if (splits > 1 && tid == 0) {
        ws[(int64_t)blockIdx.x * (D + 2) + D] = mx;
        ws[(int64_t)blockIdx.x * (D + 2) + D + 1] = sum;
    }
}

// One workgroup per unit: out = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s.
__global__ __launch_bounds__(256) void gqa_combine_kernel(GqaArgs p, const float* __restrict__ ws, int splits)
{
    const int unit = blockIdx.x;
    const GqaUnit u = gqa_unit(p, unit);
    const int D = p.D;
    const float* w = ws + (int64_t)unit * splits * (D + 2);
    float M = -__builtin_inff();
    for (int s = 0; s < splits; ++s)
        if (w[s * (D + 2) + D + 1] > 0.0f) M = fmaxf(M, w[s * (D + 2) + D]);
    float f[kGqaMaxSplits];
    float lsum = 0.0f;
    for (int s = 0; s < splits; ++s) {
        const float l = w[s * (D + 2) + D + 1];
        f[s] = l > 0.0f ? expf(w[s * (D + 2) + D] - M) : 0.0f;
        lsum = lsum + l * f[s];
    }
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    float* orow = p.out + (int64_t)(u.b * p.Sq + u.qi) * p.H * D + u.h * D;
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float o = 0.0f;
        for (int s = 0; s < splits; ++s) o = __builtin_fmaf(w[s * (D + 2) + d], f[s], o);
        orow[d] = o * inv;
    }
}

// Decode and short queries, head_dim D in {64, 128}, up to 8 query heads per kv head:
// one workgroup per (batch, kv head, query, key split) serves every query head of the
// group, so each key and value row is read once per split instead of once per query head
// (the 7B layer's 28 / 4 heads read the 2048-row history once, not 7 times). The split's
// keys go through LDS in chunks of 32 rows with an online softmax (running max, sum and
// weighted V rows per head); the partial (max, sum, row) per (unit, split) goes to the
// workspace in gqa_combine_kernel's layout, or straight to the output with one split.
constexpr int kGqaChunk = 32;
constexpr int kGqaGroupMax = 8;

template <int D>
__global__ __launch_bounds__(kGqaThreads) void gqa_group_kernel(GqaArgs p, float* __restrict__ ws, int splits)
{
    constexpr int KP = D + 4;            // padded K row: float4 reads of 16 different rows hit distinct banks
    constexpr int C4 = D / 4;            // P.V: 4-channel groups of a row
    static_assert(kGqaThreads / C4 >= kGqaGroupMax, "one P.V pass covers every head of the group");
    __shared__ __attribute__((aligned(16))) float qs[kGqaGroupMax * D];
    __shared__ __attribute__((aligned(16))) float ks[kGqaChunk * KP];
    __shared__ __attribute__((aligned(16))) float vs[kGqaChunk * D];
    __shared__ float ps[kGqaGroupMax * kGqaChunk];
    __shared__ float alpha[kGqaGroupMax];
    const int grp = p.H / p.kvH;
    const int sp = blockIdx.x % splits, ug = blockIdx.x / splits;
    const int qi = ug % p.Sq, bg = ug / p.Sq;
    const int g = bg % p.kvH, b = bg / p.kvH;
    const int tid = threadIdx.x;

    // the unit's key range (the same for every head of the group)
    int bound = p.total - 1;
    if (p.seqlens_len > 0) bound = min(bound, p.seqlens[min(b, p.seqlens_len - 1)]);
    const int q_abs = p.past + qi;
    const int k_limit = min(q_abs, bound);
    const int k_start = p.window >= 0 ? max(0, q_abs - p.window + 1) : 0;
    const int L = max(k_limit - k_start + 1, 0);
    const int j0 = k_start + (int)(((int64_t)L * sp) / splits);
    const int j1 = k_start + (int)(((int64_t)L * (sp + 1)) / splits);

    const int pos = rotary_pos(q_abs, p);
    float* const kb = p.pk + (int64_t)(b * p.kvH + g) * p.cap * D;
    float* const vb = p.pv + (int64_t)(b * p.kvH + g) * p.cap * D;
    // this (batch, kv head)'s cached rows [0, past) (the host keeps past * D * 4 below 2^31)
    const __amdgpu_buffer_rsrc_t rkc = buffer_rsrc(kb, p.past * D * 4);
    const __amdgpu_buffer_rsrc_t rvc = buffer_rsrc(vb, p.past * D * 4);
    // The new rows [past, past + Skv) of this kv head: the first workgroup of each (batch, kv
    // head) writes them to the present cache (K rotated as gqa_append_kernel does); a chunk
    // that holds one of them builds it from the input row itself, so no workgroup reads a
    // cache row another one writes. Up to kGqaGroupMax rows (every decode step) their loads
    // go out with the query rows' below and the stores follow once those have landed, so
    // the writing workgroup pays no round trip of its own; more rows take this loop first.
    const bool nwrite = qi == 0 && sp == 0 && p.Skv > 0;
    const bool nfast = p.Skv <= kGqaGroupMax;
    if (nwrite && !nfast) {
        for (int i = tid; i < p.Skv * D; i += kGqaThreads) {
            const int sr = i / D, d = i - sr * D;
            const float* krow = p.k + (int64_t)(b * p.Skv + sr) * p.kv_stride + g * D;
            const float* vrow = p.v + (int64_t)(b * p.Skv + sr) * p.kv_stride + g * D;
            kb[(int64_t)(p.past + sr) * D + d] = rotated(krow, d, rotary_pos(p.past + sr, p), p);
            vb[(int64_t)(p.past + sr) * D + d] = vrow[d];
        }
    }

    // score phase: thread (h = tid / 32, j = tid % 32); P.V phase: thread (head vh = tid / C4,
    // channels 4 vc .. 4 vc + 3 with vc = tid % C4), one 16-byte read of V per key
    const int sh = tid >> 5, sj = tid & 31;
    float m_run = -__builtin_inff(), l_run = 0.0f;   // per head, held by the 32 lanes of head sh
    const int vc = tid % C4, vh = tid / C4;
    float4 acc = float4{0.0f, 0.0f, 0.0f, 0.0f};

    // The group's query rows: their loads go first (with the cos / sin entries of their
    // rotation), the first chunk's key and value loads after them, and the rotation is
    // applied once those are in flight, so it waits for the query loads alone. The formula
    // is rotated()'s: a c - b s or b c + a s, each product rounded.
    constexpr int QPT = kGqaGroupMax * D / kGqaThreads;
    const int rot = 2 * p.rot_half;
    // the group's query rows (grp rows of D floats from this unit's query row)
    const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(p.q + (int64_t)(b * p.Sq + qi) * p.q_stride + g * grp * D, grp * D * 4);
    const __amdgpu_buffer_rsrc_t rcs = buffer_rsrc(p.do_rotary ? p.cos : p.q, p.do_rotary ? p.cache_rows * p.half * 4 : 0);
    const __amdgpu_buffer_rsrc_t rsn = buffer_rsrc(p.do_rotary ? p.sin : p.q, p.do_rotary ? p.cache_rows * p.half * 4 : 0);
    float qa[QPT], qb[QPT], qc[QPT], qn[QPT];
    bool qrot[QPT], qfirst[QPT];
#pragma unroll
    for (int t = 0; t < QPT; ++t) {
        const int i = tid + t * kGqaThreads;
        const int r = i / D, d = i - r * D;
        const bool valid = i < grp * D, rotating = p.do_rotary && d < rot;
        int j = d, i0 = d, i1 = d;
        if (rotating) {
            if (p.interleaved) {
                j = d >> 1;
                i0 = 2 * j;
                i1 = i0 + 1;
            } else {
                j = d < p.rot_half ? d : d - p.rot_half;
                i0 = j;
                i1 = j + p.rot_half;
            }
        }
        qrot[t] = rotating;
        qfirst[t] = d == i0;
        const int row = r * D;
        const int cs = rotating ? (pos * p.half + j) * 4 : kOOB;
        qa[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rq, valid ? (row + i0) * 4 : kOOB, 0, 0));
        qb[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rq, valid && rotating ? (row + i1) * 4 : kOOB, 0, 0));
        qc[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rcs, valid ? cs : kOOB, 0, 0));
        qn[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsn, valid ? cs : kOOB, 0, 0));
    }
    // The new K and V rows (nwrite && nfast: Skv * D <= QPT * kGqaThreads elements), loaded
    // the same way: element i = tid + t * kGqaThreads is channel d of new row sr, rotated at
    // position past + sr.
    const bool nload = nwrite && nfast;
    const int64_t nbase = (int64_t)b * p.Skv * p.kv_stride + g * D;
    const int nbytes = nload ? ((p.Skv - 1) * p.kv_stride + D) * 4 : 0;
    const __amdgpu_buffer_rsrc_t rnk = buffer_rsrc(p.k + nbase, nbytes), rnv = buffer_rsrc(p.v + nbase, nbytes);
    float na[QPT], nb[QPT], nc[QPT], nn[QPT], nv[QPT];
    bool nrot[QPT], nfirst[QPT];
#pragma unroll
    for (int t = 0; t < QPT; ++t) {
        const int i = tid + t * kGqaThreads;
        const int sr = i / D, d = i - sr * D;
        const bool valid = nload && i < p.Skv * D, rotating = p.do_rotary && d < rot;
        int j = d, i0 = d, i1 = d;
        if (rotating) {
            if (p.interleaved) {
                j = d >> 1;
                i0 = 2 * j;
                i1 = i0 + 1;
            } else {
                j = d < p.rot_half ? d : d - p.rot_half;
                i0 = j;
                i1 = j + p.rot_half;
            }
        }
        nrot[t] = rotating;
        nfirst[t] = d == i0;
        const int row = sr * p.kv_stride;
        const int cs = rotating ? (rotary_pos(p.past + sr, p) * p.half + j) * 4 : kOOB;
        na[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rnk, valid ? (row + i0) * 4 : kOOB, 0, 0));
        nb[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rnk, valid && rotating ? (row + i1) * 4 : kOOB, 0, 0));
        nc[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rcs, valid ? cs : kOOB, 0, 0));
        nn[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsn, valid ? cs : kOOB, 0, 0));
        nv[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rnv, valid ? (row + d) * 4 : kOOB, 0, 0));
    }

    constexpr int PER = kGqaChunk * (D / 4) / kGqaThreads;   // float4s of K (and of V) per thread
    static_assert(PER * kGqaThreads == kGqaChunk * (D / 4), "chunk shape");
    // A chunk's cached K and V rows into registers (every load in flight together,
    // branch-free: rows past the chunk or not yet in the cache read zero).
    float4 k4[PER], v4[PER];
    auto load_chunk = [&](int c0) {
        const int n = min(kGqaChunk, j1 - c0);
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i = tid + u * kGqaThreads;
            const int r = i / (D / 4), c4 = i - r * (D / 4);
            const int key = c0 + r;
            const int off = r < n && key < p.past ? (key * D + 4 * c4) * 4 : kOOB;
            k4[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rkc, off, 0, 0));
            v4[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rvc, off, 0, 0));
        }
    };
    load_chunk(j0);
    __builtin_amdgcn_sched_barrier(0);   // the first chunk's loads stay ahead of the rotation below
    // the query rows, rotated: waits for the query loads alone
#pragma unroll
    for (int t = 0; t < QPT; ++t) {
        const int i = tid + t * kGqaThreads;
        if (i < grp * D)
            qs[i] = !qrot[t] ? qa[t] : qfirst[t] ? qa[t] * qc[t] - qb[t] * qn[t] : qb[t] * qc[t] + qa[t] * qn[t];
    }
    // the new rows to the present cache (row past + sr, channel d: offset past * D + i)
    if (nload) {
#pragma unroll
        for (int t = 0; t < QPT; ++t) {
            const int i = tid + t * kGqaThreads;
            if (i < p.Skv * D) {
                kb[(int64_t)p.past * D + i] =
                    !nrot[t] ? na[t] : nfirst[t] ? na[t] * nc[t] - nb[t] * nn[t] : nb[t] * nc[t] + na[t] * nn[t];
                vb[(int64_t)p.past * D + i] = nv[t];
            }
        }
    }
    for (int c0 = j0; c0 < j1; c0 += kGqaChunk) {
        const int n = min(kGqaChunk, j1 - c0);
        if (c0 != j0) load_chunk(c0);
        // ... and a new row (at most Skv of them, at the end of the range) from the input
        if (c0 + n > p.past) {
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const int i = tid + u * kGqaThreads;
                const int r = i / (D / 4), c4 = i - r * (D / 4);
                const int key = c0 + r;
                if (r < n && key >= p.past) {
                    const int sr = key - p.past;
                    const float* krow = p.k + (int64_t)(b * p.Skv + sr) * p.kv_stride + g * D;
                    const float* vrow = p.v + (int64_t)(b * p.Skv + sr) * p.kv_stride + g * D;
                    const int kp = rotary_pos(key, p);
                    k4[u] = float4{rotated(krow, 4 * c4, kp, p), rotated(krow, 4 * c4 + 1, kp, p),
                                   rotated(krow, 4 * c4 + 2, kp, p), rotated(krow, 4 * c4 + 3, kp, p)};
                    v4[u] = float4{vrow[4 * c4], vrow[4 * c4 + 1], vrow[4 * c4 + 2], vrow[4 * c4 + 3]};
                }
            }
        }
        __syncthreads();   // the previous chunk's readers are done with ks / vs / ps
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i = tid + u * kGqaThreads;
            const int r = i / (D / 4), c4 = i - r * (D / 4);
            *reinterpret_cast<float4*>(ks + r * KP + 4 * c4) = k4[u];
            *reinterpret_cast<float4*>(vs + r * D + 4 * c4) = v4[u];
        }
        __syncthreads();
        if (sh < grp) {
            float sc = -__builtin_inff();
            if (sj < n) {
                const float* qh = qs + sh * D;
                const float* kr = ks + sj * KP;
                // four partial sums (channels d % 4), added in order at the end
                float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
#pragma unroll 8
                for (int d = 0; d < D; d += 4) {
                    const float4 q4 = *reinterpret_cast<const float4*>(qh + d);
                    const float4 kk = *reinterpret_cast<const float4*>(kr + d);
                    d0 = __builtin_fmaf(q4.x, kk.x, d0);
                    d1 = __builtin_fmaf(q4.y, kk.y, d1);
                    d2 = __builtin_fmaf(q4.z, kk.z, d2);
                    d3 = __builtin_fmaf(q4.w, kk.w, d3);
                }
                sc = ((d0 + d1) + (d2 + d3)) * p.scale;
            }
            const float cm = half_max_all(sc);   // the 32 score lanes of head sh
            const float m_new = fmaxf(m_run, cm);   // finite: the chunk holds at least one key
            const float a = expf(m_run - m_new);    // 0 on the first chunk
            const float e = sj < n ? expf(sc - m_new) : 0.0f;
            const float cs = half_sum_all(e);
            l_run = l_run * a + cs;
            m_run = m_new;
            ps[sh * kGqaChunk + sj] = e;
            if (sj == 0) alpha[sh] = a;
        }
        __syncthreads();
        if (vh < grp) {
            // per channel: o = acc * alpha, then o = fma(p_j, v_j, o) in key order
            const float a = alpha[vh];
            float4 o = float4{acc.x * a, acc.y * a, acc.z * a, acc.w * a};
            const float* ph = ps + vh * kGqaChunk;
            for (int j = 0; j < n; ++j) {
                const float pj = ph[j];
                const float4 v = *reinterpret_cast<const float4*>(vs + j * D + 4 * vc);
                o.x = __builtin_fmaf(pj, v.x, o.x);
                o.y = __builtin_fmaf(pj, v.y, o.y);
                o.z = __builtin_fmaf(pj, v.z, o.z);
                o.w = __builtin_fmaf(pj, v.w, o.w);
            }
            acc = o;
        }
    }
    // the per-head (max, sum) live in the score lanes: hand them to the P.V threads via LDS
    __syncthreads();
    if (sh < grp && sj == 0) {
        ps[sh * kGqaChunk] = m_run;
        ps[sh * kGqaChunk + 1] = l_run;
    }
    __syncthreads();
    if (vh < grp) {
        const int hh = g * grp + vh;
        const int64_t unit = ((int64_t)b * p.H + hh) * p.Sq + qi;
        const float mh = ps[vh * kGqaChunk], lh = ps[vh * kGqaChunk + 1];
        if (splits == 1) {
            const float r = lh > 0.0f ? 1.0f / lh : 0.0f;
            float* o = p.out + (int64_t)(b * p.Sq + qi) * p.H * D + hh * D + 4 * vc;
            o[0] = lh > 0.0f ? acc.x * r : 0.0f;
            o[1] = lh > 0.0f ? acc.y * r : 0.0f;
            o[2] = lh > 0.0f ? acc.z * r : 0.0f;
            o[3] = lh > 0.0f ? acc.w * r : 0.0f;
        } else {
            float* w = ws + (unit * splits + sp) * (D + 2);
            w[4 * vc] = acc.x;
            w[4 * vc + 1] = acc.y;
            w[4 * vc + 2] = acc.z;
            w[4 * vc + 3] = acc.w;
            if (vc == 0) {
                w[D] = mh;
                w[D + 1] = lh;
            }
        }
    }
}

// The splits of gqa_group_kernel meet here: one wave per (unit, 64 channels). Each lane
// issues the loads of its channel over every split and of split `lane`'s maximum and sum
// together (one round trip to memory: the workspace was written by workgroups on other
// XCDs); the maximum and the normaliser come from DPP reductions, and each lane then adds
// its channel over the splits in split order (deterministic), split s's rescale factor
// read from lane s with v_readlane. Splits past `splits` load zeros (value and factor), so
// the sum runs over all kGqaMaxSplits without a branch: a ds_bpermute per split, each
// behind a branch and its own wait, had made the merge a chain of 64 LDS round trips.
__global__ __launch_bounds__(64) void gqa_merge_kernel(GqaArgs p, const float* __restrict__ ws, int splits)
{
    const int D = p.D, slices = (D + 63) / 64;
    const int unit = blockIdx.x / slices, d = (blockIdx.x % slices) * 64 + threadIdx.x;
    const int lane = threadIdx.x;
    const GqaUnit u = gqa_unit(p, unit);
    // The unit's splits * (D + 2) floats through a buffer resource: loads past them (split
    // s >= splits, or a channel past D) return 0 without a branch.
    const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(ws + (int64_t)unit * splits * (D + 2), splits * (D + 2) * 4);
    const bool dv = d < D;
    const int dof = dv ? d * 4 : kOOB;
    float vals[kGqaMaxSplits];
#pragma unroll
    for (int s = 0; s < kGqaMaxSplits; ++s)
        vals[s] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rw, dof, s * (D + 2) * 4, 0));
    const float ml = lane < splits ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                   rw, (lane * (D + 2) + D) * 4, 0, 0))
                                   : -__builtin_inff();
    const float ll = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                   rw, lane < splits ? (lane * (D + 2) + D + 1) * 4 : kOOB, 0, 0));
    static_assert(kGqaMaxSplits == kWave, "split s's maximum and sum sit in lane s");
    const float mr = row16_max_all(ll > 0.0f ? ml : -__builtin_inff());
    const float M = fmaxf(fmaxf(lane_value(mr, 0), lane_value(mr, 16)), fmaxf(lane_value(mr, 32), lane_value(mr, 48)));
    const float f = ll > 0.0f ? expf(ml - M) : 0.0f;   // 0 for splits past `splits` (ll loads 0)
    const float lsum = lane_value(group_sum_to_last<64>(ll * f), 63);
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    float o = 0.0f;   // every lane runs the sum (lane s must be active when its factor is read)
#pragma unroll
    for (int s = 0; s < kGqaMaxSplits; ++s) o = __builtin_fmaf(vals[s], lane_value(f, s), o);
    if (dv) p.out[(int64_t)(u.b * p.Sq + u.qi) * p.H * D + u.h * D + d] = o * inv;
}

// Prefill (more than 8 queries), head_dim D in {64, 128}: flash attention on the fp32 matrix
// cores. A workgroup of 4 waves takes 64 consecutive queries of one (batch, head); wave w
// owns 16 of them. Keys go through LDS in chunks of 64 rows of K and V. Per chunk:
//   S^T = K Q^T with v_mfma_f32_16x16x4f32 (keys are the M dimension, queries N, head
//   channels K): lane l holds the scores of keys 4(l/16) + i, i < 4, of each 16-key tile for
//   query l % 16 — exactly the A-operand layout that P V needs (queries M, keys K), so the
//   probabilities never leave their registers. Channel j = 4t + i of a k step reads channel
//   16t + 4(l/16) + i, so each lane's K and Q operands of four steps are one 16-byte read.
//   Online softmax per query (max and sum over the 16-lane groups by shuffles), then
//   O += P V, O rows rescaled by exp(m_old - m_new) fetched from the lane that owns the
//   query's statistics.
// fp32 products and sums throughout: the same 1e-5-of-max|out| bar as the VALU kernels.
constexpr int kFlashQ = 64, kFlashK = 64;

template <int D>
__global__ __launch_bounds__(256, 2) void gqa_flash_kernel(GqaArgs p)
{
    typedef float floatx4_t __attribute__((ext_vector_type(4)));
    constexpr int KP = D + 4;   // padded rows: the 16-byte reads of 16 K rows, and of the 4 V rows of a step, spread over the banks
    constexpr int T = D / 16;   // k steps of four per 16-channel group
    extern __shared__ __attribute__((aligned(16))) float flash_lds[];
    float* const ks = flash_lds;
    float* const vs = flash_lds + kFlashK * KP;
    const int nqb = (p.Sq + kFlashQ - 1) / kFlashQ;
    // heaviest blocks (latest queries) first
    const int qb = nqb - 1 - (int)(blockIdx.x % nqb), hb = (int)(blockIdx.x / nqb);
    const int h = hb % p.H, b = hb / p.H, g = h / (p.H / p.kvH);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r16 = lane & 15, c = lane >> 4;
    const int q0 = qb * kFlashQ;

    int bound = p.total - 1;
    if (p.seqlens_len > 0) bound = min(bound, p.seqlens[min(b, p.seqlens_len - 1)]);
    auto k_first = [&](int qi) { return p.window >= 0 ? max(0, p.past + qi - p.window + 1) : 0; };
    auto k_last = [&](int qi) { return min(p.past + qi, bound); };

    // this lane's query (S columns) and its rotated channels 16t + 4c + i
    const int qs_i = q0 + wave * 16 + r16;
    const bool q_in = qs_i < p.Sq;
    floatx4_t qreg[T];
    {
        const float* qrow = p.q + (int64_t)(b * p.Sq + min(qs_i, p.Sq - 1)) * p.q_stride + h * D;
        const int pos = rotary_pos(p.past + qs_i, p);
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) qreg[t][i] = q_in ? rotated(qrow, 16 * t + 4 * c + i, pos, p) : 0.0f;
    }
    const int kf_q = k_first(qs_i), kl_q = q_in ? k_last(qs_i) : -1;
    // the workgroup's key range
    const int qlast = min(q0 + kFlashQ, p.Sq) - 1;
    const int kmin = k_first(q0), kmax = k_last(qlast);
    const float* kb = p.pk + (int64_t)(b * p.kvH + g) * p.cap * D;
    const float* vb = p.pv + (int64_t)(b * p.kvH + g) * p.cap * D;

    const float scale2 = p.scale * 1.44269504088896341f;   // scale * log2(e)
    float m_run = -__builtin_inff(), l_run = 0.0f;   // statistics of query r16 (in the 4 lanes of each c), base 2
    floatx4_t acc_o[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc_o[t] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // A chunk's K and V rows pass through registers: the next chunk's loads are in flight
    // while this chunk computes.
    constexpr int PER = kFlashK * (D / 4) / 256;
    float4 kr[PER], vr[PER];
    auto load_chunk = [&](int c0) {
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i4 = tid + 256 * u;
            const int r = i4 / (D / 4), c4 = i4 - r * (D / 4);
            const int key = c0 + r;
            kr[u] = vr[u] = float4{0.0f, 0.0f, 0.0f, 0.0f};
            if (key < p.total) {
                kr[u] = *reinterpret_cast<const float4*>(kb + (int64_t)key * D + 4 * c4);
                vr[u] = *reinterpret_cast<const float4*>(vb + (int64_t)key * D + 4 * c4);
            }
        }
    };
    const int cfirst = (kmin / kFlashK) * kFlashK;
    if (cfirst <= kmax) load_chunk(cfirst);
    for (int c0 = cfirst; c0 <= kmax; c0 += kFlashK) {
        __syncthreads();   // the previous chunk's readers are done
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i4 = tid + 256 * u;
            const int r = i4 / (D / 4), c4 = i4 - r * (D / 4);
            *reinterpret_cast<float4*>(ks + r * KP + 4 * c4) = kr[u];
            *reinterpret_cast<float4*>(vs + r * KP + 4 * c4) = vr[u];
        }
        __syncthreads();
        if (c0 + kFlashK <= kmax) load_chunk(c0 + kFlashK);
        // S^T tiles: 4 x (16 keys x 16 queries), the four tiles' chains interleaved
        floatx4_t st[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) st[kt] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float4 kv[4];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
                kv[kt] = *reinterpret_cast<const float4*>(ks + (kt * 16 + r16) * KP + 4 * c + 16 * t);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) st[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[kt].x, qreg[t][0], st[kt], 0, 0, 0);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) st[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[kt].y, qreg[t][1], st[kt], 0, 0, 0);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) st[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[kt].z, qreg[t][2], st[kt], 0, 0, 0);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) st[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[kt].w, qreg[t][3], st[kt], 0, 0, 0);
        }
        // scale, mask (only chunks that cross a query's key range), chunk maximum of query r16.
        // Scores are kept in base 2 (times scale * log2(e)): the softmax is then
        // 2^(s - max) with the hardware exp2 (v_exp_f32, 1 ulp), the same weights as
        // e^(scale q.k - max) to about 1e-7 relative, well inside the 1e-5 bar.
        const bool full = __all(c0 >= kf_q && c0 + kFlashK - 1 <= kl_q);
        float cm = -__builtin_inff();
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = c0 + kt * 16 + 4 * c + i;
                const bool ok = full || (key >= kf_q && key <= kl_q);
                const float sc = ok ? st[kt][i] * scale2 : -__builtin_inff();
                st[kt][i] = sc;
                cm = fmaxf(cm, sc);
            }
        cm = fmaxf(cm, xor16_value(cm));   // the query's 4 lanes (rows c) of the wave
        cm = fmaxf(cm, xor32_value(cm));
        const float m_new = fmaxf(m_run, cm);
        const bool none = m_new == -__builtin_inff();   // no key of this query so far
        const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
        float ls = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = none ? 0.0f : __builtin_amdgcn_exp2f(st[kt][i] - m_new);
                st[kt][i] = e;
                ls = ls + e;
            }
        ls = ls + xor16_value(ls);
        ls = ls + xor32_value(ls);
        l_run = l_run * alpha + ls;
        m_run = m_new;
        // rescale O rows (queries 4c + i of the wave) by their alpha
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float ai = __shfl(alpha, 4 * c + i);
#pragma unroll
            for (int t = 0; t < T; ++t) acc_o[t][i] = acc_o[t][i] * ai;
        }
        // O += P V: A = P (queries x keys, from st), B = V (keys x channels). Output tile t
        // column r16 is channel T r16 + t, so a lane's B operands of one key row are T
        // consecutive floats (16-byte reads).
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float* vrow = vs + (kt * 16 + 4 * c + i) * KP + T * r16;
                float4 vv[T / 4];
#pragma unroll
                for (int w = 0; w < T / 4; ++w) vv[w] = *reinterpret_cast<const float4*>(vrow + 4 * w);
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const float4& v4 = vv[t >> 2];
                    const float bv = (t & 3) == 0 ? v4.x : (t & 3) == 1 ? v4.y : (t & 3) == 2 ? v4.z : v4.w;
                    acc_o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(st[kt][i], bv, acc_o[t], 0, 0, 0);
                }
            }
    }
    // out rows: queries 4c + i of the wave, channels T r16 + t (T consecutive floats per lane)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float li = __shfl(l_run, 4 * c + i);
        const int qo = q0 + wave * 16 + 4 * c + i;
        if (qo < p.Sq) {
            float* orow = p.out + (int64_t)(b * p.Sq + qo) * p.H * D + h * D + T * r16;
            const float inv = li > 0.0f ? 1.0f / li : 0.0f;
#pragma unroll
            for (int w = 0; w < T / 4; ++w)
                *reinterpret_cast<float4*>(orow + 4 * w) = float4{acc_o[4 * w][i] * inv, acc_o[4 * w + 1][i] * inv,
                                                                  acc_o[4 * w + 2][i] * inv, acc_o[4 * w + 3][i] * inv};
        }
    }
}

}  // namespace msnb
