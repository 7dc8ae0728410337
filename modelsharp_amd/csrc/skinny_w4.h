// skinny_w4.h — small-M INT4 GEMV on the matrix cores at fp32-level accuracy
// (M <= 16, block size 128, K a multiple of 128).
//
// Y[M,N] = A[M,K] * W^T with W = (q - zp) * s. Per weight row n and block b (128 k):
//     Y[m][n] += s[n][b] * sum_{k in b} A[m][k] * (q[n][k] - zp[n][b]).
// The inner sums run on v_mfma_f32_16x16x32_f16 without losing fp32 accuracy:
//   * q - zp is a small integer, exact in fp16 (the 0x6400 magic and one packed
//     subtract, as in the prefill kernel's dequant, without the scale);
//   * A is split per row m and block b into A = 2^e * (hi + lo), hi = fp16(A 2^-e),
//     lo = fp16(A 2^-e - hi), with e chosen so the block's max |A| 2^-e lies in
//     [2^14, 2^15). Every product hi (q - zp) and lo (q - zp) is exact in fp32, and
//     hi + lo carries A to about 2^-22 of the block's max;
//   * the block sums (fp32, accumulated by the MFMAs) are multiplied by 2^e (exact) and
//     by s, and added to the running sum in fp32.
// So the arithmetic is the GEMV's (exact products, fp32 sums, the scale applied per
// block); only the activations' last bits below 2^-22 of the block max are dropped.
//
// Work mapping. A workgroup (4 waves) owns kSkinnyRows weight rows and a range of at
// most kSkinnyNB blocks; each wave owns 16 * kSkinnyNF of the rows. The workgroup
//   1. issues its activation loads, then the scales and zero points of its rows (the
//      NB lanes of a row read its NB blocks' values together and hand them on by
//      ds_bpermute), then every weight load of every wave (all blocks in flight at
//      once: a block costs a wave 4 * kSkinnyNF registers, the activations live in LDS);
//   2. converts the activations of its K range to hi / lo / 2^e straight into LDS, in
//      the MFMA operand order, while the weights are in flight;
//   3. per block and fragment: lane (n = lane % 16, s = lane / 16) holds the 16-byte
//      chunk s of its row's 64-byte block and feeds dword j of it to MFMA step j
//      (j = 0..3): step j covers k = 32 s + 8 j + [0, 8) for s = 0..3, so the four
//      steps cover the block, and the activations in LDS are laid out to match (lane
//      (m, s) of step j reads 16 contiguous bytes, a whole step 1 KB);
//   4. `ksw` workgroups split a row tile's blocks and meet in one of two ways (both
//      deterministic: partial sums are added in index order):
//        - ksw <= kSkinnyHandoffMax: through per-workgroup slots (rows m < M only), the
//          last to arrive summing the slots (the arrival counters reset themselves);
//        - wider splits: workgroup kw stores its sums to slice kw of a [ksw][M][N]
//          workspace with plain stores, and skinny_reduce_kernel adds the slices into Y
//          (the kernel boundary orders the two launches).
//      The hand-off's store completion, arrival atomic and slot loads form one latency
//      chain at the end of each tile that grows with ksw; the separate reduce costs a
//      launch. Measured (graph-timed, K=4096/N=11008, ksw 8, M = 4 / 16): hand-off 13.7 /
//      15.9 us, reduce 14.4 / 16.9; K=11008/N=4096, ksw 22: hand-off 17.0 / 20.8, reduce
//      14.7 / 17.0.
// The activation permutation within an 8-k group is k0,k4,k1,k5,k2,k6,k3,k7: the order
// in which the dequant produces fp16 pairs from one dword of packed nibbles.
#pragma once
#include "nbits_device.h"
#include "mfma_w4.h"

namespace msnb {

constexpr int kSkinnyMT = 16;                            // MFMA rows: M padded to 16
constexpr int kSkinnyNF = 2;                             // 16-row MFMA fragments per wave
constexpr int kSkinnyRows = 4 * 16 * kSkinnyNF;          // weight rows per workgroup
constexpr int kSkinnyNB = 4;                             // blocks per workgroup, at most
constexpr int kSkinnyStepBytes = 1024;                   // one MFMA step's activations (hi or lo)
constexpr int kSkinnyBlockBytes = 4 * 2 * kSkinnyStepBytes;   // one block: 4 steps x (hi, lo)
constexpr int kSkinnySlot = kSkinnyMT * kSkinnyRows;     // floats per workgroup slot (hand-off)
constexpr int kSkinnyHandoffMax = 8;                     // widest K split that uses the hand-off

struct SkinnyParams {
    const uint8_t* b;          // [N][row_bytes]
    const float* scales;       // [N][nb]
    const uint8_t* zp;         // [N][zrb] or nullptr (zp = 8)
    const float* a;            // [M][K]
    float* y;                  // [M][N]
    float* part;               // [ksw][slice4 * 4] partial sums of Y (ksw > kSkinnyHandoffMax), or nullptr
    int slice4;                // float4 per slice: M * N rounded up
    float* slots;              // [row tiles][ksw][kSkinnySlot] (1 < ksw <= kSkinnyHandoffMax)
    int* sync;                 // [row tiles] arrival counters, zero between launches (idem)
    int row_bytes, M, N, K, nb, zrb;
    int ksw;                   // workgroups per row tile: ksw * kSkinnyNB >= K / 128, ksw <= K / 128
};

// The 8 codes of MFMA step j of a lane's 128-k block as four fp16 pairs (q - zp), in the
// order (k_t, k_{t+4}) of the permuted activations, exact (|q - zp| <= 255). 4-bit codes:
// dword j of the lane's 16-byte chunk; 8-bit codes (B8): dwords 2j, 2j + 1 of its 32
// bytes, whose byte t and byte t of the next dword v_perm puts side by side.
template <bool B8>
__device__ __forceinline__ half8_t skinny_step_codes(uint32_t d0, uint32_t d1, h2_t z2)
{
    uint32_t o[4];
    if constexpr (B8) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
            o[t] = as_u32(as_h2(and_or(__builtin_amdgcn_perm(d1, d0, (uint32_t)(((4 + t) << 16) | t)), 0x00FF00FFu,
                                       kHalfMagic)) - z2);
    } else {
        (void)d1;
        o[0] = as_u32(as_h2(and_or(d0, 0x000F000Fu, kHalfMagic)) - z2);
        o[1] = as_u32(as_h2(and_or(d0 >> 4, 0x000F000Fu, kHalfMagic)) - z2);
        o[2] = as_u32(as_h2(and_or(d0 >> 8, 0x000F000Fu, kHalfMagic)) - z2);
        o[3] = as_u32(as_h2(and_or(d0 >> 12, 0x000F000Fu, kHalfMagic)) - z2);
    }
    return __builtin_bit_cast(half8_t, u32x4_t{o[0], o[1], o[2], o[3]});
}

template <int QPB, bool B8>
__global__ __launch_bounds__(256) void skinny_w4_kernel(SkinnyParams p)
{
    static_assert(QPB == 1 || QPB == 2 || QPB == 4, "block sizes 128, 64, 32");
    constexpr bool PS = QPB > 1;   // a scale per 32-k step (bs 32, 64), not per 128-k block
    constexpr int CW = B8 ? 2 : 1; // 16-byte code chunks per lane and block (8-bit: 32 codes in 32 bytes)
    constexpr int ZB = B8 ? 8 : 4; // bits per zero point
    constexpr int NF = kSkinnyNF, NB = kSkinnyNB;
    __shared__ __attribute__((aligned(16))) uint32_t lds_a[NB * kSkinnyBlockBytes / 4];
    __shared__ __attribute__((aligned(16))) float lds_e[NB * kSkinnyMT];

    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int ln = lane & 15, ls = lane >> 4;
    const int rt = blockIdx.x / p.ksw, kw = blockIdx.x - rt * p.ksw;
    const int G = p.K >> 7;
    const int g0 = (int)((int64_t)kw * G / p.ksw), g1 = (int)((int64_t)(kw + 1) * G / p.ksw);
    const int cnt = g1 - g0;                                  // 1 .. NB blocks
    const int n0 = rt * kSkinnyRows + wave * 16 * NF;         // this wave's first row

    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(p.a, p.M * p.K * 4);
    const __amdgpu_buffer_rsrc_t rb_ = buffer_rsrc(p.b, p.N * p.row_bytes);
    const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(p.scales, p.N * p.nb * 4);
    const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(p.zp ? (const void*)p.zp : (const void*)p.scales,
                                                  p.zp ? p.N * p.zrb : 0);

    // ---- 1. loads: activations first (they are consumed first), then the weights ----
    // Activation pass i: row m = 4 i + gi / 4 and block lg = gi % 4 of the range, where
    // gi = tid / 16 is a 16-lane group and lane pl = tid % 16 takes k = 8 pl .. 8 pl + 7
    // of the block (two 16-byte loads). Only rows m < M and blocks lg < cnt are read.
    const int gi = tid >> 4, pl = tid & 15;
    u32x4_t av[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * i + (gi >> 2), lg = gi & 3;
        const bool ok = m < p.M && lg < cnt;
        const int off = (m * p.K + (g0 + lg) * 128 + 8 * pl) * 4;
        av[i][0] = __builtin_amdgcn_raw_buffer_load_b128(ra, ok ? off : kOOB, 0, 0);
        av[i][1] = __builtin_amdgcn_raw_buffer_load_b128(ra, ok ? off + 16 : kOOB, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);

    // Scales and zero points of the wave's rows and blocks: for fragment f, lane l takes
    // (row 16 f + l / NB, block l % NB), so the NB neighbouring lanes of a row read its
    // blocks together (one line request per row and instruction; a load per lane, block
    // and fragment made four times as many, and cost about 3 us of a 24 MB launch). The
    // lane that computes (row 16 f + ln, block lg) reads them from lane NB ln + lg.
    static_assert(16 * NB == kWave, "one lane per (row, block) of a fragment");
    // With QPB > 1 quantization blocks per 128-k block (block sizes 32, 64), lane (ln, ls)
    // of fragment f loads instead the QPB scales of its row's block ls (one aligned 8- or
    // 16-byte load: nb is a multiple of QPB) and their zero-point nibbles, and the lane that
    // computes step j of block lg takes them from lane (ln, lg).
    float sv[NF][QPB];
    uint32_t zv[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        if constexpr (PS) {
            const int n = n0 + 16 * f + ln, q0 = (g0 + ls) * QPB;
            const bool ok = n < p.N && ls < cnt;
            const int so = ok ? (n * p.nb + q0) * 4 : kOOB;
            // the QPB zero points: 4-bit nibbles (2 or 1 bytes at q0 / 2), 8-bit bytes
            // (4 or 2 bytes at q0; zrb = nb, a multiple of QPB, keeps them aligned)
            const int zo = ok ? n * p.zrb + (B8 ? q0 : q0 / 2) : kOOB;
            if constexpr (QPB == 4) {
                const float4 v = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsc, so, 0, 0));
                sv[f][0] = v.x;
                sv[f][1] = v.y;
                sv[f][2] = v.z;
                sv[f][3] = v.w;
                zv[f] = B8 ? __builtin_amdgcn_raw_buffer_load_b32(rz, zo, 0, 0)
                           : __builtin_amdgcn_raw_buffer_load_b16(rz, zo, 0, 0);
            } else {
                const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rsc, so, 0, 0));
                sv[f][0] = __builtin_bit_cast(float, v.x);
                sv[f][1] = __builtin_bit_cast(float, v.y);
                zv[f] = B8 ? __builtin_amdgcn_raw_buffer_load_b16(rz, zo, 0, 0)
                           : __builtin_amdgcn_raw_buffer_load_b8(rz, zo, 0, 0);
            }
        } else {
            const int n = n0 + 16 * f + lane / NB, blk = lane % NB, g = g0 + blk;
            const bool ok = n < p.N && blk < cnt;
            sv[f][0] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(rsc, ok ? n * p.nb * 4 + g * 4 : kOOB, 0, 0));
            zv[f] = __builtin_amdgcn_raw_buffer_load_b8(rz, ok ? n * p.zrb + (B8 ? g : g >> 1) : kOOB, 0, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    int cbase[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        const int n = n0 + 16 * f + ln;
        cbase[f] = n < p.N ? n * p.row_bytes + ls * 16 * CW : kOOB;
    }
    // One load group per block, issued in block order, so computing block lg waits only
    // for its own group (the scheduling barriers keep the groups apart).
    u32x4_t c[NB][NF][CW];
#pragma unroll
    for (int lg = 0; lg < NB; ++lg) {
        const int g = g0 + lg;
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const bool ok = lg < cnt && cbase[f] != kOOB;
#pragma unroll
            for (int h = 0; h < CW; ++h)
                c[lg][f][h] = __builtin_amdgcn_raw_buffer_load_b128(rb_, ok ? cbase[f] + g * 64 * CW + 16 * h : kOOB, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- 2. activations -> LDS: hi / lo fp16 in the MFMA operand order, 2^e per row/block ----
    // LDS layout: block lg, step j, part (0 hi, 1 lo): 1 KB of 64 16-byte chunks; the
    // chunk of (s, m), holding k = 32 s + 8 j + (0,4,1,5,2,6,3,7), sits at position
    // 16 s + (m ^ c) with c = 8 (s & 1) + 2 j + part. The swizzle keeps both sides free
    // of bank conflicts: a 16-lane group converting one row writes 16 different
    // positions (per part), and an MFMA step's 64 lanes read 64 different ones.
    // Rows m >= M hold zeros (their MFMA rows then add nothing) and 2^e = 0.
#pragma unroll
    for (int u = 0; u < NB * kSkinnyBlockBytes / (16 * 256); ++u) {
        const int gc = tid + 256 * u, step = gc >> 6, pc = gc & 63, s = pc >> 4;
        const int m = (pc & 15) ^ (((s & 1) << 3) | (((step >> 1) & 3) << 1) | (step & 1));
        if (m >= p.M) *reinterpret_cast<u32x4_t*>(&lds_a[gc * 4]) = u32x4_t{0u, 0u, 0u, 0u};
    }
    if (tid < NB * kSkinnyMT && (tid & 15) >= p.M) lds_e[tid] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (4 * i >= p.M) break;
        const int m = 4 * i + (gi >> 2), lg = gi & 3;
        const float4 v0 = __builtin_bit_cast(float4, av[i][0]), v1 = __builtin_bit_cast(float4, av[i][1]);
        const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        float mx = 0.0f;
#pragma unroll
        for (int r = 0; r < 8; ++r) mx = fmaxf(mx, fabsf(v[r]));
        mx = row16_max_all(mx);   // the 16 lanes of this row and block
        // mx in [2^(E-1), 2^E) with E = frexp exponent; 2^-e with e = E - 15 brings it
        // into [2^14, 2^15) (an all-zero block gets e = -15 and stays zero).
        const int e = __builtin_amdgcn_frexp_expf(mx) - 15;
        if (m < p.M && lg < cnt) {
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                // the pair (k = 8 pl + t, 8 pl + 4 + t): chunk order k0,k4,k1,k5,...
                const float x0 = __builtin_amdgcn_ldexpf(v[t], -e), x1 = __builtin_amdgcn_ldexpf(v[t + 4], -e);
                const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
                const _Float16 l0 = (_Float16)(x0 - (float)h0), l1 = (_Float16)(x1 - (float)h1);
                hw[t] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                lw[t] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
            }
            // k = 8 pl .. 8 pl + 7 of the block is step j, lane group s: k = 32 s + 8 j
            // per 128-k block scale (the codes' 16-byte chunk s is one step's k range of
            // lane group s), k = 32 j + 8 s with a scale per 32-k step (after the 4 x 4
            // transpose of the code dwords, step j is quantization block j).
            const int s = PS ? (pl & 3) : (pl >> 2), j = PS ? (pl >> 2) : (pl & 3), c = ((s & 1) << 3) | (j << 1);
            const int base = (lg * 4 + j) * 2 * kSkinnyStepBytes + s * 256;
            *reinterpret_cast<u32x4_t*>(&lds_a[(base + (m ^ c) * 16) / 4]) = u32x4_t{hw[0], hw[1], hw[2], hw[3]};
            *reinterpret_cast<u32x4_t*>(&lds_a[(base + kSkinnyStepBytes + (m ^ (c | 1)) * 16) / 4]) =
                u32x4_t{lw[0], lw[1], lw[2], lw[3]};
            if (pl == 0) lds_e[lg * kSkinnyMT + m] = __builtin_amdgcn_ldexpf(1.0f, e);
        }
    }
    __syncthreads();

    // ---- 3. blocks ----
    floatx4_t acc[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[f] = floatx4_t{};
    const uint32_t zdef = p.zp ? 0u : (B8 ? 128u : 8u);   // without zero points the zp loads read zeros
    // This lane's chunk (s = ls, m = ln) of each step j and part, within a block's 8 KB.
    int aoff[4][2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int pt = 0; pt < 2; ++pt)
            aoff[j][pt] = (j * 2 + pt) * kSkinnyStepBytes + ls * 256 + (ln ^ (((ls & 1) << 3) | (j << 1) | pt)) * 16;
    }
#pragma unroll
    for (int lg = 0; lg < NB; ++lg) {
        if (lg >= cnt) break;
        const float4 e4 = *reinterpret_cast<const float4*>(&lds_e[lg * kSkinnyMT + 4 * ls]);
        const float ev[4] = {e4.x, e4.y, e4.z, e4.w};
        if constexpr (PS) {
            // Transpose the code dwords across the four 16-lane rows (lane (ln, s) had
            // dword j of quantization block s; after it, dword s of block j): step j is
            // block j. The permlane swaps exchange whole rows, lane ln stays lane ln. With
            // 8-bit codes a step is a pair of dwords (2 j, 2 j + 1): the even and the odd
            // dwords are transposed alike.
            uint32_t t[NF][CW][4];
#pragma unroll
            for (int f = 0; f < NF; ++f) {
#pragma unroll
                for (int h = 0; h < CW; ++h) {
                    uint32_t d[4];   // dword i (4-bit) or 2 i + h (8-bit) of the lane's codes, i = 0..3
                    if constexpr (B8) {
                        d[0] = h ? c[lg][f][0].y : c[lg][f][0].x;
                        d[1] = h ? c[lg][f][0].w : c[lg][f][0].z;
                        d[2] = h ? c[lg][f][1].y : c[lg][f][1].x;
                        d[3] = h ? c[lg][f][1].w : c[lg][f][1].z;
                    } else {
                        d[0] = c[lg][f][0].x;
                        d[1] = c[lg][f][0].y;
                        d[2] = c[lg][f][0].z;
                        d[3] = c[lg][f][0].w;
                    }
                    const auto a0 = __builtin_amdgcn_permlane32_swap(d[0], d[2], false, false);
                    const auto a1 = __builtin_amdgcn_permlane32_swap(d[1], d[3], false, false);
                    const auto b0 = __builtin_amdgcn_permlane16_swap(a0[0], a1[0], false, false);
                    const auto b1 = __builtin_amdgcn_permlane16_swap(a0[1], a1[1], false, false);
                    t[f][h][0] = b0[0];
                    t[f][h][1] = b0[1];
                    t[f][h][2] = b1[0];
                    t[f][h][3] = b1[1];
                }
            }
            const int src = (ln + 16 * lg) * 4;   // ds_bpermute byte address of lane (ln, lg)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int qj = j * QPB / 4;   // quantization block of step j within block lg
                const half8_t ah = *reinterpret_cast<const half8_t*>(&lds_a[(lg * kSkinnyBlockBytes + aoff[j][0]) / 4]);
                const half8_t al = *reinterpret_cast<const half8_t*>(&lds_a[(lg * kSkinnyBlockBytes + aoff[j][1]) / 4]);
#pragma unroll
                for (int f = 0; f < NF; ++f) {
                    const float sc =
                        __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, sv[f][qj])));
                    const uint32_t zq = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)zv[f]);
                    const uint32_t zp = ((zq >> (ZB * qj)) & ((1u << ZB) - 1)) + zdef;
                    const h2_t z2 = as_h2(kHalfMagic | (zp << 16) | zp);
                    const half8_t bq = skinny_step_codes<B8>(t[f][0][j], t[f][CW - 1][j], z2);
                    const floatx4_t th = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq, floatx4_t{}, 0, 0, 0);
                    const floatx4_t tl = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bq, floatx4_t{}, 0, 0, 0);
                    // step sums for activation row m = 4 ls + v and weight row n0 + 16 f + ln:
                    // times 2^e[m] (exact) and the step's scale, into the running sum
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[f][v] = __builtin_fmaf((th[v] + tl[v]) * ev[v], sc, acc[f][v]);
                }
            }
        } else {
            floatx4_t th[NF], tl[NF];
            uint32_t zb[NF];
            float sc[NF];
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                th[f] = floatx4_t{};
                tl[f] = floatx4_t{};
                const int src = (NB * ln + lg) * 4;   // ds_bpermute byte address of lane NB ln + lg
                sc[f] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, sv[f][0])));
                const uint32_t zq = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)zv[f]);
                const uint32_t zp = (B8 ? (zq & 0xFFu) : ((zq >> (((g0 + lg) & 1) * 4)) & 0x0Fu)) + zdef;
                zb[f] = kHalfMagic | (zp << 16) | zp;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const half8_t ah = *reinterpret_cast<const half8_t*>(&lds_a[(lg * kSkinnyBlockBytes + aoff[j][0]) / 4]);
                const half8_t al = *reinterpret_cast<const half8_t*>(&lds_a[(lg * kSkinnyBlockBytes + aoff[j][1]) / 4]);
#pragma unroll
                for (int f = 0; f < NF; ++f) {
                    // step j: dword j of the 16-byte chunk (4-bit), dwords 2 j, 2 j + 1 of the 32 bytes (8-bit)
                    const u32x4_t& cw = c[lg][f][B8 ? (j >> 1) : 0];
                    const uint32_t d0 = B8 ? ((j & 1) ? cw.z : cw.x) : (j == 0 ? cw.x : j == 1 ? cw.y : j == 2 ? cw.z : cw.w);
                    const uint32_t d1 = B8 ? ((j & 1) ? cw.w : cw.y) : 0u;
                    const half8_t bq = skinny_step_codes<B8>(d0, d1, as_h2(zb[f]));
                    th[f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq, th[f], 0, 0, 0);
                    tl[f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bq, tl[f], 0, 0, 0);
                }
            }
            // th / tl[f][v]: block sums for activation row m = 4 ls + v and weight row
            // n0 + 16 f + ln; times 2^e[m] (exact) and s[n], into the running sum.
#pragma unroll
            for (int f = 0; f < NF; ++f) {
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[f][v] = __builtin_fmaf((th[f][v] + tl[f][v]) * ev[v], sc[f], acc[f][v]);
            }
        }
    }

    // ---- 4. output: Y itself, slice kw of the partial sums (summed by skinny_reduce_kernel),
    // or the hand-off ----
    if (p.ksw == 1 || p.part) {
        float* const out = p.ksw == 1 ? p.y : p.part + (int64_t)kw * p.slice4 * 4;
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const int n = n0 + 16 * f + ln;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int m = 4 * ls + v;
                if (m < p.M && n < p.N) out[(int64_t)m * p.N + n] = acc[f][v];
            }
        }
        return;
    }
    // Slots [m][kSkinnyRows] (rows m < M), written through to device scope and read
    // back by the last arriver with device-coherent loads: the hand-off needs no L2
    // write-back or invalidate, only the order (every slot store has completed before
    // the barrier that precedes the arrival; the last arriver's loads follow its count).
    const __amdgpu_buffer_rsrc_t rsl = buffer_rsrc(p.slots, (int)gridDim.x * kSkinnySlot * 4);
    const int own = (rt * p.ksw + kw) * kSkinnySlot;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        const int col = wave * 16 * NF + 16 * f + ln;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int m = 4 * ls + v;
            const float val = acc[f][v];   // a scalar first: a bit cast of a vector element reads element 0
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, val), rsl,
                                                  m < p.M ? (own + m * kSkinnyRows + col) * 4 : kOOB, 0,
                                                  kDeviceCoherent);
        }
    }
    wait_vmem_order_only_release();
    __syncthreads();
    __shared__ int arrival;
    if (tid == 0) arrival = __hip_atomic_fetch_add(p.sync + rt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrival != p.ksw - 1) return;
    wait_vmem_order_only_acquire();
    if (tid == 0) __hip_atomic_store(p.sync + rt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Thread t sums the 4 columns at e_i = 4 (t + 256 i) of every slot (i < kI), rows
    // e_i / kSkinnyRows = (t + 256 i) / 32, i.e. 8 i .. 8 i + 7: only i < ceil(M / 8) carry
    // rows of A. All its slot loads (ksw <= kSkinnyHandoffMax per i) are in flight
    // together, then added per element in slot order.
    constexpr int kI = kSkinnySlot / (4 * 256);
    const int first = rt * p.ksw * kSkinnySlot;
#pragma unroll
    for (int i = 0; i < kI; ++i) {
        const int e = 4 * (tid + 256 * i), m = e / kSkinnyRows, col = e - m * kSkinnyRows;
        if (8 * i >= p.M) break;
        u32x4_t sl[kSkinnyHandoffMax];
#pragma unroll
        for (int w = 0; w < kSkinnyHandoffMax; ++w)
            sl[w] = __builtin_amdgcn_raw_buffer_load_b128(
                rsl, w < p.ksw && m < p.M ? (first + w * kSkinnySlot + e) * 4 : kOOB, 0, kDeviceCoherent);
        if (m >= p.M) continue;
        float4 tot = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < kSkinnyHandoffMax; ++w) {
            if (w < p.ksw) {
                const float4 v = __builtin_bit_cast(float4, sl[w]);
                tot.x += v.x;
                tot.y += v.y;
                tot.z += v.z;
                tot.w += v.w;
            }
        }
        const float tv[4] = {tot.x, tot.y, tot.z, tot.w};
        const int nb0 = rt * kSkinnyRows + col;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if (nb0 + t < p.N) p.y[(int64_t)m * p.N + nb0 + t] = tv[t];
        }
    }
}

// Y[j] = sum over the ksw slices of part[w][j], in slice order (deterministic), for the
// n = M * N elements of Y; thread i takes elements 4i .. 4i + 3 with every slice's load
// in flight at once (up to kSkinnyRedBatch per round trip).
constexpr int kSkinnyRedBatch = 32;
__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float* __restrict__ part, float* __restrict__ y,
                                                            int n, int slice4, int ksw)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= slice4) return;
    const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(part, ksw * slice4 * 16);
    float4 t = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int w0 = 0; w0 < ksw; w0 += kSkinnyRedBatch) {
        u32x4_t v[kSkinnyRedBatch];
#pragma unroll
        for (int u = 0; u < kSkinnyRedBatch; ++u)
            v[u] = __builtin_amdgcn_raw_buffer_load_b128(rp, w0 + u < ksw ? ((w0 + u) * slice4 + i) * 16 : kOOB, 0, 0);
#pragma unroll
        for (int u = 0; u < kSkinnyRedBatch; ++u) {
            if (w0 + u < ksw) {
                const float4 f = __builtin_bit_cast(float4, v[u]);
                t.x += f.x;
                t.y += f.y;
                t.z += f.z;
                t.w += f.w;
            }
        }
    }
    const float tv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int c = 0; c < 4; ++c)
        if (4 * i + c < n) y[4 * i + c] = tv[c];
}

}  // namespace msnb
