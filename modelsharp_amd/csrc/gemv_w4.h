// gemv_w4.h — dequant-fused INT4 GEMV for 1 <= M <= 4 (the decode path), for one
// weight matrix or a group of up to four that share the activations.
//
// Work mapping (wave64-first):
//   * A workgroup of WAVES waves owns ROWS = (64/G) * (WAVES/KW) consecutive output
//     rows n. Inside a wave, G lanes share a row and R = 64/G rows sit side by
//     side; KW waves split the same rows' K. A step advances each lane by
//     SPAN = G*KW chunks of 32 codes (one 16-byte load per chunk), so one
//     wave-wide code load reads R contiguous segments of G*16 bytes of packed B
//     in the reference layout B[n][K/2].
//   * The whole activation panel A[0..M)[0..K) is staged once per workgroup in
//     LDS (odd k pre-divided by 16; kChunkStride4 float4 per chunk).
//   * Load order is the design: every vector-memory load returns in issue order,
//     so the activation loads go first, then NB batches of U steps of codes,
//     scales and zero points, and only then is A written to LDS. The staging
//     therefore waits for the activations alone while the weight stream is
//     already in flight. Loads are unconditional (a lane with no chunk at a step
//     loads from kOOB: zero, no memory request), which keeps the compiler's
//     wait counts exact; sched_barrier keeps the scheduler from reordering the
//     three groups. Addresses are one per-lane base plus compile-time step
//     strides (L = log2 chunks per block is a template parameter).
//   * End: the G partial sums of a row meet in a butterfly over the G lanes,
//     the KW wave partials in LDS (fixed orders: deterministic); one lane stores.
// Arithmetic per chunk (32 codes q_k, zero point zp, scale s):
//   A code masked into the mantissa of the fp16 1024.0 reads as 1024 + q (code bits
//   0-3) or 1024 + 16q (bits 4-7); one packed subtract of 1024 + zp (resp.
//   1024 + 16 zp) leaves q - zp (resp. 16 (q - zp)) exactly. With the activations
//   staged as a_k (even k) and a_k / 16 (odd k) — exact powers of two — one
//   v_fma_mix_f32 adds exactly a_k (q_k - zp) into an fp32 sum. Per activation row m,
//       blk = sum_k a_k (q_k - zp),   acc += s * blk,
//   the dot product with the dequantized weights W = (q - zp) s with the scale applied
//   once per block: the reference's sum in another order, with no cancelling terms
//   (its error stays within eps * sum_k |a_k (q_k - zp) s|). For M <= 2 the 32
//   products go into two partial sums (shorter dependency chains).
// HBM traffic is the algorithmic minimum: every byte of B, scales and zero
// points is read once; A is read once per workgroup (L2-resident).
#pragma once
#include "nbits_device.h"

namespace msnb {

// One launch serves up to kGemvMaxOps weight matrices that share the activations A
// and K (the projections of one input: q/k/v, gate/up); op i owns workgroups
// [first, next op's first).
constexpr int kGemvMaxOps = 4;
struct GemvOp {
    const uint8_t* b;        // [N][row_bytes] packed codes (reference layout)
    const float* scales;     // [N][nb]
    const uint8_t* zp;       // [N][zrb] packed nibbles, or nullptr (zp = 8)
    float* y;                // [M][N]
    int N;
    int first;               // first workgroup of this op
};
struct GemvParams {
    GemvOp op[kGemvMaxOps];
    int nops;
    const float* a;          // [M][K]
    int row_bytes;           // nb * block_size / 2
    int K;
    int C;                   // K / 32 chunks per row
    int nb, zrb;
    // NORM launches (M = 1): A = SkipRMSNorm(nx + nskip) * ngamma, computed by every workgroup
    // from nx, nskip and ngamma; workgroup 0 writes nx + nskip to nsum (when not null) and
    // the normed activations to nout.
    const float* nx;
    const float* nskip;
    const float* ngamma;
    float* nsum;
    float* nout;
    float neps;
};

// Uniform choice among the op table's entries (selects on a wave-uniform index, so the
// table stays in the kernel arguments).
template <typename T>
__device__ __forceinline__ T op_field(int oi, T v0, T v1, T v2, T v3)
{
    return oi == 0 ? v0 : oi == 1 ? v1 : oi == 2 ? v2 : v3;
}

// SW (SwiGLU): ops 0 and 1 are the gate and up projections of one input (same N); the first
// half of the row-waves computes gate rows, the second half the same rows of up, and the
// epilogue stores H = (g * (1 / (1 + exp(-g)))) * u into op 1's output (the SiLU-Mul of
// silu_mul_kernel, with its roundings), so the gate and up rows never leave the workgroup.
//
// NORM (M = 1): the activations are SkipSimplifiedLayerNormalization's output, computed in
// the workgroup's staging instead of read: t = x + skip, then A = (t * inv) * gamma with
// inv = 1 / sqrt(sum t^2 / K + eps). Each workgroup stages t * gamma (two threads per
// chunk, 16 values each; the host checks 2 C <= threads) and its share of sum t^2, and
// applies inv to its sums before they are stored: y = inv * sum_k W_k (t_k gamma_k), the
// same dot product in another order. The staging loads are consumed before the weight
// stream is issued, so the stream's registers are not held beside them (issuing the first
// weight batch ahead of the staging measured no faster: the 7B q+k+v with its norm 7.9 ->
// 8.5 us). The staging reads three vectors where gemv_w4 reads one, which every workgroup
// pays in L2 bandwidth: the 7B gate+up+SiLU launch with its norm takes 22.6 us against 19.9
// without (the norm's own launch 4.1 us). Workgroup 0 also
// writes t (the residual stream) and (t * inv) * gamma; neither may overlap x or skip,
// which the other workgroups are still reading (checked by the host).
template <int M, int G, int KW, int U, int L, int WAVES, int RL, int NB, bool SW = false, bool NORM = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_w4_kernel(GemvParams p)
{
    static_assert(!NORM || M == 1, "the fused norm serves one row of activations");
    static_assert(NB >= 2 && NB <= 4, "two to four load batches in flight");
    constexpr int R = kWave / G;
    constexpr int WR = WAVES / KW;
    static_assert(!SW || WR % 2 == 0, "SwiGLU splits the row-waves between gate and up");
    constexpr int WRO = SW ? WR / 2 : WR;   // row-waves per op
    constexpr int ROWS0 = R * WRO;     // rows of one layer; a lane owns RL rows, ROWS0 apart
    constexpr int ROWS = RL * ROWS0;   // rows per workgroup (of each op with SW)
    constexpr int SPAN = G * KW;
    constexpr int BSPAN = SPAN >> L;   // blocks per step
    static_assert((BSPAN << L) == SPAN && (BSPAN & 1) == 0, "a step covers an even number of whole blocks");
    static_assert(WR * KW == WAVES, "KW must divide WAVES");
    extern __shared__ float4 lds_a4[];  // [M][C][kChunkStride4]
    __shared__ float red[KW > 1 ? KW : 1][(SW ? 2 : 1) * ROWS][M];
    __shared__ float swx[SW ? ROWS : 1][M];   // SW: the gate rows, handed to the up waves
    __shared__ float nred[NORM ? WAVES : 1];  // NORM: the waves' sums of t^2

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int g = lane % G, r = lane / G;
    const int wk = wave % KW, wr = wave / KW;
    const int rl = (SW ? wr % WRO : wr) * R + r;
    const int bid = blockIdx.x;
    // The op is uniform over a wave (per workgroup without SW, per wave with it): read
    // through the first lane so its buffer descriptors stay scalar.
    const int oi = SW ? __builtin_amdgcn_readfirstlane(wr / WRO)
                      : (p.nops > 1 && bid >= p.op[1].first) + (p.nops > 2 && bid >= p.op[2].first) +
                            (p.nops > 3 && bid >= p.op[3].first);
    const uint8_t* const ob = op_field(oi, p.op[0].b, p.op[1].b, p.op[2].b, p.op[3].b);
    const float* const osc = op_field(oi, p.op[0].scales, p.op[1].scales, p.op[2].scales, p.op[3].scales);
    const uint8_t* const ozp = op_field(oi, p.op[0].zp, p.op[1].zp, p.op[2].zp, p.op[3].zp);
    float* const oy = op_field(oi, p.op[0].y, p.op[1].y, p.op[2].y, p.op[3].y);
    const int N = op_field(oi, p.op[0].N, p.op[1].N, p.op[2].N, p.op[3].N);
    const int first = SW ? 0 : op_field(oi, p.op[0].first, p.op[1].first, p.op[2].first, p.op[3].first);
    // Row slot rl + j * ROWS0 of this workgroup is row n0 + j * ROWS0; slots past N idle.
    const int n0 = (bid - first) * ROWS + rl;
    bool vrow[RL];
#pragma unroll
    for (int j = 0; j < RL; ++j) vrow[j] = n0 + j * ROWS0 < N;
    const int C = p.C;
    const int nsteps = (C + SPAN - 1) / SPAN;
    const int lofs = wk * G + g;                       // chunk offset within a step
    const int nvalid = lofs < C ? (C - lofs + SPAN - 1) / SPAN : 0;

    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(p.a, M * p.K * 4);
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(ob, N * p.row_bytes);
    const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(osc, N * p.nb * 4);
    const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(ozp ? (const void*)ozp : (const void*)osc, ozp ? N * p.zrb : 0);

    // ---- 1. activation chunks: first in the load queue -------------------------------
    const int na = M * C;
    const int idx = threadIdx.x;                      // M * C <= 64 * WAVES (checked by the host)
    const int am = idx / C, ac = idx - am * C;
    const int aoff = idx < na ? (am * p.K + ac * 32) * 4 : kOOB;
    float4 av[8];
    float4 xv[4], kv[4], gv[4];   // NORM: half chunk idx of x, skip and gamma
    if constexpr (NORM) {
        // Half chunk idx (values 16 idx .. 16 idx + 15) of x, skip and gamma, consumed (below)
        // before the weight stream is issued.
        const int ho = idx < 2 * C ? idx * 64 : kOOB;
        const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(p.nx, p.K * 4), rk = buffer_rsrc(p.nskip, p.K * 4),
                                     rg = buffer_rsrc(p.ngamma, p.K * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            xv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, ho, 16 * j, 0));
            kv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, ho, 16 * j, 0));
            gv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rg, ho, 16 * j, 0));
        }
    } else {
        // The chunk's 16-byte offsets ride in the scalar offset, so kOOB itself is never
        // added to in int arithmetic (the hardware adds them as unsigned 32-bit values, and
        // kOOB + 112 still lies past every buffer).
#pragma unroll
        for (int j = 0; j < 8; ++j)
            av[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ra, aoff, 16 * j, 0));
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. weight stream: NB batches of U steps in flight ----------------------------
    // An idle row slot loads from kOOB (zeros, no memory request); its sums are not stored.
    int bbase[RL], sbase[RL], zbase[RL];
#pragma unroll
    for (int j = 0; j < RL; ++j) {
        const int nl = vrow[j] ? n0 + j * ROWS0 : 0;
        bbase[j] = nl * p.row_bytes + lofs * 16;
        sbase[j] = nl * p.nb * 4 + (lofs >> L) * 4;
        zbase[j] = nl * p.zrb + ((lofs >> L) >> 1);
    }
    const int zshift = ((lofs >> L) & 1) * 4;
    struct Batch {
        u32x4_t q[RL][U];
        float s[RL][U];
        uint8_t z[RL][U];   // bytes: a widened copy could be hoisted ahead of the batch's wait
    };
    // The codes are read once per call, each 128-byte line whole by one load of G lanes:
    // non-temporal loads keep them from displacing the activations, outputs, scales and
    // zero points in L2 / MALL. Scale and zero-point lines serve several steps of a row, so
    // they stay cached (non-temporal there too refetched them). Measured on the 7B decode
    // layer: 46.2 -> 43.4 us per step of 4 launches; the gate+up launch 20.1 -> 18.2 us.
    auto load = [&](Batch& bt, int k0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = k0 + u;
#pragma unroll
            for (int j = 0; j < RL; ++j) {
                const bool ok = k < nvalid && vrow[j];
                bt.q[j][u] = __builtin_amdgcn_raw_buffer_load_b128(rb, ok ? bbase[j] + k * (SPAN * 16) : kOOB, 0,
                                                                   kNonTemporal);
                bt.s[j][u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                           rsc, ok ? sbase[j] + k * (BSPAN * 4) : kOOB, 0, 0));
                bt.z[j][u] = __builtin_amdgcn_raw_buffer_load_b8(rz, ok ? zbase[j] + k * (BSPAN / 2) : kOOB, 0,
                                                                 0);
            }
        }
    };
    // A ring of NB batches of U steps: batch b holds steps k0 + b U .. + U - 1; each is
    // refilled with the steps NB U further on as soon as it has been reduced, so between
    // (NB - 1) U and NB U steps per lane are always in flight.
    Batch bt[NB];
    if constexpr (NORM) {
        // t = x + skip, t * gamma staged, the thread's share of sum t^2 (in the order of
        // skip_rmsnorm_kernel's f4sq); then the weight batches.
        const bool hv = idx < 2 * C;
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 t = float4{xv[j].x + kv[j].x, xv[j].y + kv[j].y, xv[j].z + kv[j].z, xv[j].w + kv[j].w};
            ss = ss + t.x * t.x;
            ss = ss + t.y * t.y;
            ss = ss + t.z * t.z;
            ss = ss + t.w * t.w;
            if (bid == 0 && hv && p.nsum) reinterpret_cast<float4*>(p.nsum)[4 * idx + j] = t;
            if (hv)
                lds_a4[(idx >> 1) * kChunkStride4 + (idx & 1) * 4 + j] =
                    stage_odd16(float4{t.x * gv[j].x, t.y * gv[j].y, t.z * gv[j].z, t.w * gv[j].w});
        }
        ss = group_sum_to_last<64>(ss);
        if ((idx & (kWave - 1)) == kWave - 1) nred[idx / kWave] = ss;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < NB; ++b) load(bt[b], b * U);
    } else {
#pragma unroll
        for (int b = 0; b < NB; ++b) load(bt[b], b * U);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 3. stage A: odd k divided by 16 (exact), matching 16 (q - zp) of the dequant ----
    if constexpr (!NORM) {
        if (idx < na) {
            float4* dst = &lds_a4[idx * kChunkStride4];
#pragma unroll
            for (int j = 0; j < 8; ++j) dst[j] = stage_odd16(av[j]);
        }
    }
    __syncthreads();
    // NORM: inv from the waves' sums of t^2 in wave order (every thread, the same value)
    float inv = 1.0f;
    if constexpr (NORM) {
        float sst = nred[0];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) sst = sst + nred[w];
        inv = 1.0f / __builtin_sqrtf(sst / (float)p.K + p.neps);
    }

    float acc[RL][M];
#pragma unroll
    for (int j = 0; j < RL; ++j) {
#pragma unroll
        for (int m = 0; m < M; ++m) acc[j][m] = 0.0f;
    }
    auto reduce = [&](const Batch& bt, int k0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = k0 + u;
            if (k < nvalid) {
                const int c = k * SPAN + lofs;
                // Walk the chunk one code dword (8 codes, two float4 of activations) at a time:
                // each LDS read of activations serves the lane's RL rows, and only one dword's
                // code pairs per row are live. For M <= 2 even and odd dwords feed two partial
                // sums (shorter dependency chains); otherwise one chain in dword order.
                constexpr int NP = M <= 2 ? 2 : 1;
                float t[RL][M][NP];
#pragma unroll
                for (int j = 0; j < RL; ++j) {
#pragma unroll
                    for (int m = 0; m < M; ++m) {
#pragma unroll
                        for (int q = 0; q < NP; ++q) t[j][m][q] = 0.0f;
                    }
                }
                h2_t zb[RL], zb16[RL];
#pragma unroll
                for (int j = 0; j < RL; ++j) {
                    const uint32_t zp = ozp ? ((uint32_t)bt.z[j][u] >> zshift) & 0x0Fu : 8u;
                    zb[j] = zp_half2(zp);
                    zb16[j] = zp16_half2(zp);
                }
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    uint32_t pr[RL][4];
#pragma unroll
                    for (int j = 0; j < RL; ++j) {
                        const uint32_t qd = d == 0 ? bt.q[j][u].x : d == 1 ? bt.q[j][u].y : d == 2 ? bt.q[j][u].z : bt.q[j][u].w;
                        diffs8(qd, zb[j], zb16[j], pr[j]);
                    }
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const float4* arow = &lds_a4[(m * C + c) * kChunkStride4];
                        const float4 a0 = arow[2 * d], a1 = arow[2 * d + 1];
#pragma unroll
                        for (int j = 0; j < RL; ++j) t[j][m][d % NP] = dot8(pr[j], a0, a1, t[j][m][d % NP]);
                    }
                }
#pragma unroll
                for (int m = 0; m < M; ++m) {
#pragma unroll
                    for (int j = 0; j < RL; ++j) {
                        const float blkacc = NP == 2 ? t[j][m][0] + t[j][m][NP - 1] : t[j][m][0];
                        acc[j][m] = __builtin_fmaf(bt.s[j][u], blkacc, acc[j][m]);
                    }
                }
            }
        }
    };
    // The exit leaves the whole loop (goto): a `break` out of the inner loop alone gives the
    // compiler a path back to the loop head on which the last batch was not refilled, and
    // its wait counts at the head then drain every load (vmcnt(0)) on every iteration.
    for (int k0 = 0;; k0 += NB * U) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (k0 + b * U >= nsteps) goto steps_done;
            reduce(bt[b], k0 + b * U);
            load(bt[b], k0 + (b + NB) * U);
        }
    }
steps_done:

    // ---- 4. combine: G lanes (DPP scan), then KW waves (LDS, in wave order) -----------
    // The G lanes' sums end in lane g == G - 1 of each group.
#pragma unroll
    for (int j = 0; j < RL; ++j) {
#pragma unroll
        for (int m = 0; m < M; ++m) acc[j][m] = group_sum_to_last<G>(acc[j][m]);
    }
    const int ro = SW ? oi * ROWS : 0;   // this op's rows in red
    if constexpr (KW > 1) {
        if (g == G - 1) {
#pragma unroll
            for (int j = 0; j < RL; ++j) {
#pragma unroll
                for (int m = 0; m < M; ++m) red[wk][ro + j * ROWS0 + rl][m] = acc[j][m];
            }
        }
        __syncthreads();
        if (wk == 0 && g == G - 1) {
#pragma unroll
            for (int j = 0; j < RL; ++j) {
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    float s = red[0][ro + j * ROWS0 + rl][m];
#pragma unroll
                    for (int w = 1; w < KW; ++w) s += red[w][ro + j * ROWS0 + rl][m];
                    acc[j][m] = s;
                }
            }
        }
    }
    if constexpr (SW) {
        // the gate rows to LDS; the up waves then store (g * sigmoid(g)) * u
        if (oi == 0 && wk == 0 && g == G - 1) {
#pragma unroll
            for (int j = 0; j < RL; ++j) {
#pragma unroll
                for (int m = 0; m < M; ++m) swx[j * ROWS0 + rl][m] = NORM ? acc[j][m] * inv : acc[j][m];
            }
        }
        __syncthreads();
        if (oi == 1 && wk == 0 && g == G - 1) {
#pragma unroll
            for (int j = 0; j < RL; ++j) {
                if (vrow[j]) {
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const float x = swx[j * ROWS0 + rl][m];
                        const float sg = 1.0f / (1.0f + expf(-x));
                        const float u = NORM ? acc[j][m] * inv : acc[j][m];
                        oy[(int64_t)m * N + n0 + j * ROWS0] = (x * sg) * u;
                    }
                }
            }
        }
    } else if (wk == 0 && g == G - 1) {
#pragma unroll
        for (int j = 0; j < RL; ++j) {
            if (vrow[j]) {
#pragma unroll
                for (int m = 0; m < M; ++m)
                    oy[(int64_t)m * N + n0 + j * ROWS0] = NORM ? acc[j][m] * inv : acc[j][m];
            }
        }
    }
    // NORM: workgroup 0 writes the normed activations, (t * inv) * gamma (the roundings of
    // skip_rmsnorm_kernel), from x, skip and gamma read again.
    if constexpr (NORM) {
        if (bid == 0 && idx < 2 * C) {
            const float4* x4 = reinterpret_cast<const float4*>(p.nx) + 4 * idx;
            const float4* k4 = reinterpret_cast<const float4*>(p.nskip) + 4 * idx;
            const float4* g4 = reinterpret_cast<const float4*>(p.ngamma) + 4 * idx;
            float4* o4 = reinterpret_cast<float4*>(p.nout) + 4 * idx;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 x = x4[j], k = k4[j], gm = g4[j];
                const float4 t = float4{x.x + k.x, x.y + k.y, x.z + k.z, x.w + k.w};
                o4[j] = float4{(t.x * inv) * gm.x, (t.y * inv) * gm.y, (t.z * inv) * gm.z, (t.w * inv) * gm.w};
            }
        }
    }
}

// Launch configurations of gemv_w4_kernel (one instantiation each per M and L).
struct GemvConfig {
    int waves, G, KW, U, RL, NB;
};
constexpr GemvConfig kGemvConfigs[] = {
    {4, 16, 1, 2, 1, 2},  {4, 16, 1, 4, 1, 2},  {4, 32, 1, 4, 1, 2},  {4, 64, 1, 2, 1, 2},  {4, 16, 4, 2, 1, 2},
    {4, 32, 2, 2, 1, 2},  {8, 32, 1, 4, 1, 2},  {8, 16, 2, 4, 1, 2},  {8, 16, 4, 2, 1, 2},  {16, 16, 4, 2, 1, 2},
    {16, 32, 2, 2, 1, 2}, {4, 16, 1, 2, 2, 2},  {4, 16, 1, 4, 2, 2},  {4, 32, 1, 2, 2, 2},  {4, 64, 1, 2, 2, 2},
    {8, 16, 2, 2, 2, 2},  {4, 16, 1, 1, 2, 2},  {8, 64, 1, 1, 2, 2},  {16, 16, 4, 1, 1, 2},
};
constexpr int kNumGemvConfigs = sizeof(kGemvConfigs) / sizeof(kGemvConfigs[0]);
constexpr int kGemvMaxM = 4;

}  // namespace msnb
