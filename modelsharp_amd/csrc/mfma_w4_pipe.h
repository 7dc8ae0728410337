// mfma_w4_pipe.h — INT4 MatMulNBits prefill GEMM on the CDNA4 matrix cores with a
// buffer->LDS load pipeline (M > 16, block size 32, K a multiple of 128), optionally
// with each tile's K range split over two workgroups.
//
// Y[M,N] = A[M,K] * W[N,K]^T, W = (q - zp) * s dequantized in-kernel.
//
// Two launches per call:
//   a_rows_f16_kernel  A (fp32) -> fp16 workspace, row m scaled by an exact power of
//                    two 2^-e[m] that brings its max |A| into [2^14, 2^15) (so no
//                    finite fp32 row overflows fp16, and small rows stay out of its
//                    subnormal range), each 8-k group stored in the order
//                    (k0,k4),(k1,k5),(k2,k6),(k3,k7) — the order in which the
//                    weight dequant below produces its codes, so both MFMA
//                    operands carry the same permutation of k (a dot product does
//                    not depend on the order of its terms). The epilogue
//                    multiplies row m's sums by 2^e[m] (exact).
//   mfma_w4_pipe_kernel
//     * A 256x256 output tile per workgroup: 4 waves in a 2x2 layout, each wave
//       128x128 as 4x4 v_mfma_f32_32x32x16_f16 fragments accumulating in AGPRs.
//       A step is 32 k (one block of 32 codes per weight row).
//     * Every global load of the main loop is a buffer->LDS load
//       (buffer_load_{ushort,dwordx4} ... lds) issued from inline asm, so no vector
//       register waits on memory and the compiler inserts no conservative
//       s_waitcnt for them; each wait is an explicit vmcnt count that follows
//       from the issue order below (which is why the loop is unrolled by 4).
//         - A: 4 LDS stages of one step (256 rows x 64 B, 16-byte chunks XOR-
//           swizzled per row against bank conflicts), issued 3 steps ahead;
//         - weights: per group of 4 steps, 64 B of codes, 16 B of scales and
//           2 zero-point bytes per row, in three buffers, issued two groups
//           ahead, so a row's codes for 4 steps are one contiguous 64-byte request.
//     * Dequant: each lane owns one weight row of the tile (the rows its own wave
//       loaded, so only a wave-local wait is needed). It turns 32 codes into fp16
//       with packed-half math — the code in the mantissa of 1024.0 minus
//       (1024 + zp) is exactly q - zp, times the block scale rounded to fp16 —
//       and writes them to a double-buffered fp16 weight tile.
//     * Software pipeline inside a step: the MFMA operands of each half step are
//       read from LDS under the MFMAs of the other half, and the dequant's VALU
//       work and LDS traffic are interleaved one by one with the MFMAs
//       (sched_group_barrier), since a wave keeps about 5 VALU instructions in
//       the shadow of one 32-cycle MFMA.
//     * One barrier per step. Tile order is XCD-aware (workgroup b runs on XCD
//       b % 8; each XCD walks an m-major range of tiles, sharing A panels in L2).
//     * Split K (for launches with too few tiles to fill the CUs, or for the tiles of
//       a last, partly filled round): the two halves of a split tile (whole groups
//       of 4 steps each) are neighbouring work items; the first to finish writes its
//       partial sums through to a workspace slot and raises a flag, the second adds the
//       slot to its own sums and stores Y once (deterministic: fp32 a + b == b + a).
// Numerics: A rounded once to fp16 after its row's power-of-two scaling;
// W = fl16((q - zp) * fl16(s)); products exact, sums fp32, then the row's 2^e.
// W stays in fp16 range only for scales whose nonzero magnitudes lie in
// [2^-14, 4364]: the library checks that once per weights handle and sends other
// weights to mfma_w4 (fp32 scales, exact integer weights).
#pragma once
#include "mfma_w4.h"
#include <type_traits>

namespace msnb {

struct PipeParams {
    const uint8_t* b;
    const float* scales;
    const uint8_t* zp;       // nullptr: zp = 8
    const _Float16* a16;     // [M][K] fp16, permuted within 8-k groups, row m scaled by 2^-rexp[m]
    const int* rexp;         // [M] row exponents of a16
    float* y;                // [M][N]
    int row_bytes, M, N, K, C, nb, zrb;
    int tiles_m, tiles_n;
    // Tiles [0, full) run whole; each tile from `full` on has its K range split over two
    // workgroups. Workgroup b runs on XCD x = b % 8: its first xv work items (b / 8 < xv)
    // are the halves of split tiles full + x*xv/2 .., the next xu whole tiles x*xu ..
    int full, xu, xv;
    int* sync;               // split tile t: sync[2 (t - full) ..] arrival tag and ready flag, zero
    float* part;             // split tile t: slot t - full of kPipeBM * kPipeBN partial sums
    int epoch;               // this launch's nonzero tag in sync (tells overlapping launches apart)
    int spin_limit;          // polls of the first half's flag before the second half gives up
    int* err;                // set to a nonzero code when a split tile's hand-off fails
};

// Codes written to PipeParams::err.
constexpr int kPipeErrTimeout = 1;   // the first half's flag did not come within the bound
constexpr int kPipeErrOverlap = 2;   // another launch holds the tile's counters

constexpr int kPipeBM = 256, kPipeBN = 256;
// LDS of a launch: NA stages of A (one step each), NG weight groups (codes, scales, zero
// points of 4 steps), two fp16 weight tiles, then the tile's row exponents (1 KB); the
// kernel declares no static LDS. 4-bit codes: 4 stages and 3 groups, all 160 KB of a CU;
// 8-bit codes (128 bytes per row and group): 3 stages and 2 groups (155 KB).
template <bool B8>
struct PipeLds {
    static constexpr int NA = B8 ? 3 : 4, NG = B8 ? 2 : 3;
    static constexpr int CROW = B8 ? 128 : 64;   // code bytes per row and group
    static constexpr int A_ST = kPipeBM * 64, CG = kPipeBN * CROW, SG = kPipeBN * 16, ZG = kPipeBN * 4;
    static constexpr int OFF_A = 0, OFF_C = NA * A_ST, OFF_S = OFF_C + NG * CG, OFF_Z = OFF_S + NG * SG,
                         OFF_B = OFF_Z + NG * ZG, OFF_E = OFF_B + 2 * kPipeBN * 64;
    static constexpr int BYTES = OFF_E + kPipeBM * 4;
    static_assert(BYTES <= 160 * 1024, "the pipelined prefill's LDS exceeds a CU's");
};
// Base offset of a row beyond the matrix: above every buffer the kernel reads
// (the host checks each is smaller), so loads from it return zero.
constexpr int kPipeFar = 0x40000000;

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi)
{
    return __builtin_bit_cast(uint32_t, h2_t{(_Float16)lo, (_Float16)hi});
}

__device__ __forceinline__ float max_abs8(const float4& lo, const float4& hi)
{
    return fmaxf(fmaxf(fmaxf(fabsf(lo.x), fabsf(lo.y)), fmaxf(fabsf(lo.z), fabsf(lo.w))),
                 fmaxf(fmaxf(fabsf(hi.x), fabsf(hi.y)), fmaxf(fabsf(hi.z), fabsf(hi.w))));
}

// Exponent e of a row whose largest magnitude is mx: mx * 2^-e lies in [2^14, 2^15)
// (mx in [2^(E-1), 2^E) with E = frexp exponent, e = E - 15). Rows that are all zero,
// or hold an inf (fmaxf skips NaN), take e = 0: their sums are zero or non-finite
// whatever the scaling.
__device__ __forceinline__ int row_exponent(float mx)
{
    return (mx > 0.0f && mx <= 3.402823466e38f) ? __builtin_amdgcn_frexp_expf(mx) - 15 : 0;
}

// Largest value of x over the workgroup of 256 threads, in every thread.
__device__ __forceinline__ float block256_max(float x, float* red4)
{
    x = row16_max_all(x);
    x = fmaxf(x, xor16_value(x));
    x = fmaxf(x, xor32_value(x));
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) red4[wave] = x;
    __syncthreads();
    return fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3]));
}

__device__ __forceinline__ u32x4_t pack_group(const float4& lo, const float4& hi, int e)
{
    auto sc = [&](float v) { return __builtin_amdgcn_ldexpf(v, -e); };
    return u32x4_t{pack_h2(sc(lo.x), sc(hi.x)), pack_h2(sc(lo.y), sc(hi.y)), pack_h2(sc(lo.z), sc(hi.z)),
                   pack_h2(sc(lo.w), sc(hi.w))};
}

// fp32 -> fp16, one workgroup of 256 threads per row m: the row's max |A| gives its
// exponent e (row_exponent), stored in rexp[m]; the row is written times 2^-e (exact)
// in the permuted 8-k group order above. Thread t takes groups t, t + 256, ...: with
// R > 0 the row's R * 256 >= K / 8 groups are held in registers between the max and
// the conversion (one read of A); R == 0 reads the row twice (the second read hits L2).
template <int R>
__global__ __launch_bounds__(256) void a_rows_f16_kernel(const float* __restrict__ a, uint32_t* __restrict__ o,
                                                         int* __restrict__ rexp, int K)
{
    __shared__ float red4[4];
    const int m = blockIdx.x, tid = threadIdx.x, G8 = K >> 3;
    const float4* src = reinterpret_cast<const float4*>(a + (int64_t)m * K);
    u32x4_t* dst = reinterpret_cast<u32x4_t*>(o) + (int64_t)m * G8;
    float mx = 0.0f;
    if constexpr (R > 0) {
        float4 lo[R], hi[R];
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const int i = tid + 256 * u;
            lo[u] = i < G8 ? src[2 * i] : float4{0.0f, 0.0f, 0.0f, 0.0f};
            hi[u] = i < G8 ? src[2 * i + 1] : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < R; ++u) mx = fmaxf(mx, max_abs8(lo[u], hi[u]));
        const int e = row_exponent(block256_max(mx, red4));
        if (tid == 0) rexp[m] = e;
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const int i = tid + 256 * u;
            if (i < G8) dst[i] = pack_group(lo[u], hi[u], e);
        }
    } else {
        for (int i = tid; i < G8; i += 256) mx = fmaxf(mx, max_abs8(src[2 * i], src[2 * i + 1]));
        const int e = row_exponent(block256_max(mx, red4));
        if (tid == 0) rexp[m] = e;
        for (int i = tid; i < G8; i += 256) dst[i] = pack_group(src[2 * i], src[2 * i + 1], e);
    }
}

// The register depth a_rows_f16_kernel takes for rows of K (a multiple of 8) values.
inline int a_rows_depth(int K)
{
    const int per = (K / 8 + 255) / 256;
    for (int r : {1, 2, 4, 6, 8, 12})
        if (per <= r) return r;
    return 0;
}

inline void launch_a_rows_f16(const float* a, uint32_t* o, int* rexp, int M, int K, hipStream_t stream)
{
    const dim3 grid((unsigned)M), block(256);
    switch (a_rows_depth(K)) {
        case 1: hipLaunchKernelGGL(a_rows_f16_kernel<1>, grid, block, 0, stream, a, o, rexp, K); break;
        case 2: hipLaunchKernelGGL(a_rows_f16_kernel<2>, grid, block, 0, stream, a, o, rexp, K); break;
        case 4: hipLaunchKernelGGL(a_rows_f16_kernel<4>, grid, block, 0, stream, a, o, rexp, K); break;
        case 6: hipLaunchKernelGGL(a_rows_f16_kernel<6>, grid, block, 0, stream, a, o, rexp, K); break;
        case 8: hipLaunchKernelGGL(a_rows_f16_kernel<8>, grid, block, 0, stream, a, o, rexp, K); break;
        case 12: hipLaunchKernelGGL(a_rows_f16_kernel<12>, grid, block, 0, stream, a, o, rexp, K); break;
        default: hipLaunchKernelGGL(a_rows_f16_kernel<0>, grid, block, 0, stream, a, o, rexp, K); break;
    }
}

// fp16 weights of one dword of codes in the order (k0,k4),(k1,k5),(k2,k6),(k3,k7).
__device__ __forceinline__ void dequant8_f16(uint32_t x, h2_t zb, h2_t s2, uint32_t (&o)[4])
{
    const uint32_t m = kHalfMagic;
    o[0] = as_u32((as_h2(and_or(x, 0x000F000Fu, m)) - zb) * s2);
    o[1] = as_u32((as_h2(and_or(x >> 4, 0x000F000Fu, m)) - zb) * s2);
    o[2] = as_u32((as_h2(and_or(x >> 8, 0x000F000Fu, m)) - zb) * s2);
    o[3] = as_u32((as_h2(and_or(x >> 12, 0x000F000Fu, m)) - zb) * s2);
}

// Eight 8-bit codes (d0 = codes 0..3, d1 = codes 4..7, one byte each) as four fp16 pairs
// (k_t, k_{t+4}), t = 0..3, the order of dequant8_f16's pairs (and of the permuted A):
// v_perm gathers byte t of d0 and byte t of d1 into halves 0 and 1, v_and_or puts them
// under the exponent of 1024.0 (1024 + q exactly), then (1024 + q) - (1024 + zp) = q - zp
// exactly (|q - zp| <= 255) and one rounding to fp16 of (q - zp) * fl16(s).
__device__ __forceinline__ void dequant8_f16_b8(uint32_t d0, uint32_t d1, h2_t zb, h2_t s2, uint32_t (&o)[4])
{
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t pr = __builtin_amdgcn_perm(d1, d0, (uint32_t)(((4 + t) << 16) | t));
        o[t] = as_u32((as_h2(and_or(pr, 0x00FF00FFu, kHalfMagic)) - zb) * s2);
    }
}

typedef __attribute__((address_space(3))) uint8_t lds_byte_t;
__device__ __forceinline__ uint32_t lds_address(const void* p) { return (uint32_t)(uintptr_t)(lds_byte_t*)p; }

// buffer -> LDS loads: lane i's bytes land at LDS m0 + 16*i (x4) or m0 + 4*i (ushort).
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, int voff, int soff, uint32_t m0v)
{
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "{m0}"(m0v) : "memory");
}
__device__ __forceinline__ void lds_load4(__amdgpu_buffer_rsrc_t r, int voff, int soff, uint32_t m0v)
{
    asm volatile("buffer_load_dword %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "{m0}"(m0v) : "memory");
}
__device__ __forceinline__ void lds_load2(__amdgpu_buffer_rsrc_t r, int voff, int soff, uint32_t m0v)
{
    asm volatile("buffer_load_ushort %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "{m0}"(m0v) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 16-byte chunk slot of k-chunk j in row r: conflict-free for 8- and 16-row passes.
__device__ __forceinline__ int pipe_slot(int r, int j) { return j ^ (((r >> 2) & 3) ^ (r & 2)); }

// One work item of the pipelined launch: a whole tile, or one K half of a split tile.
struct PipeItem {
    int tile, c0, nsteps, m0, n0;   // steps [c0, c0 + nsteps) of tile (m0, n0)
    bool split;
};

// Decodes workgroup blockIdx.x's work item; false when the grid's padding has none.
// Each XCD walks a contiguous range of split tiles, whose two K halves are neighbouring
// items of the same XCD, then a contiguous (m-major) range of whole tiles. Split halves
// go first: their hand-off (slot write, slot read, Y write) then overlaps the whole
// tiles' MFMAs instead of being the launch's last, exposed burst of stores (measured at
// M=2048, K=4096, 88 split and 256 whole tiles: 203.0-204.2 -> 194.4-195.1 us).
__device__ __forceinline__ bool pipe_item(const PipeParams& p, PipeItem& it)
{
    const int tiles = p.tiles_m * p.tiles_n;
    const int xcd = blockIdx.x % kXcds, xj = blockIdx.x / kXcds;
    int kpart;
    if (xj >= p.xv) {
        it.tile = xcd * p.xu + (xj - p.xv);
        kpart = 0;
        it.split = false;
        if (it.tile >= p.full) return false;
    } else {
        const int q = xj;
        it.tile = p.full + xcd * (p.xv >> 1) + (q >> 1);
        kpart = q & 1;
        it.split = true;
        if (it.tile >= tiles) return false;
    }
    // Both halves are whole groups of 4 steps.
    const int groups = p.C >> 2, g0 = it.split ? kpart * (groups >> 1) : 0;
    it.c0 = 4 * g0;
    it.nsteps = 4 * (!it.split ? groups : kpart == 0 ? (groups >> 1) : groups - g0);
    it.m0 = (it.tile / p.tiles_n) * kPipeBM;
    it.n0 = (it.tile % p.tiles_n) * kPipeBN;
    return true;
}

// Stores a work item's 256x256 accumulators (4 waves in 2x2, each 4x4 fragments of
// v_mfma_f32_32x32x16 layout) into Y, through the split-K hand-off for split tiles.
// erow[r] (LDS) is the exponent of tile row r: Y = acc * 2^erow (exact).
// xs (LDS) holds two ints of workgroup-wide state for the split-K hand-off.
__device__ __forceinline__ void pipe_epilogue(const PipeParams& p, const PipeItem& it, floatx16_t (&acc)[4][4],
                                              const int* erow, int* xs)
{
    constexpr int BM = kPipeBM, BN = kPipeBN, FM = 4, FN = 4;
    // Lane indices from an opaque copy of the thread id: the compiler cannot share the
    // epilogue's address terms with the main loop's and keep them live (spilled) across it.
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & (kWave - 1), wave = tid / kWave;
    const int wm = wave & 1, wn = wave >> 1, lr = lane & 31, lh = lane >> 5;
    const int m0 = it.m0, n0 = it.n0, tile = it.tile;
    const bool split = it.split;
    // Exponent of accumulator row v of fragment row block i (four rows per LDS read).
    auto row_exp = [&](int i, int v) {
        const int4 e4 = *reinterpret_cast<const int4*>(&erow[wm * 128 + 32 * i + 4 * lh + 8 * (v >> 2)]);
        const int s = v & 3;
        return s == 0 ? e4.x : s == 1 ? e4.y : s == 2 ? e4.z : e4.w;
    };
    // acc[i][j][v] is Y[row][col], col = lane % 32, row = 8*(v/4) + 4*(lane/32) + v%4.
    // Stores go through a buffer resource with an offset that has bit 30 set outside the
    // valid rows/columns (every destination is smaller than 2^30 bytes, checked by the
    // host): such stores are dropped, so the epilogue has no branches. The destination
    // is runtime data: the tile (rb, cb) of an ld-wide matrix with rl x cl valid entries.
    // SCALE applies the row exponents (the final Y); the split slot holds raw sums.
    auto store_tile = [&](__amdgpu_buffer_rsrc_t rd, int ld, int rb, int cb, int rl, int cl, auto cpol, auto scale) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int row0 = wm * 128 + 32 * i + 4 * lh;
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int col = wn * 128 + 32 * j + lr;
                const uint32_t base = ((uint32_t)(rb + row0) * (uint32_t)ld + (uint32_t)(cb + col)) * 4u;
                const int cfree = cl - 1 - col;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int rv = 8 * (v >> 2) + (v & 3);
                    const uint32_t outside = (uint32_t)(((rl - 1 - row0 - rv) | cfree) >> 31);   // all ones outside
                    const int off = (int)((base + (uint32_t)(rv * 4) * (uint32_t)ld) | (outside & (uint32_t)kPipeFar));
                    // Read the accumulator with an AGPR operand: used as a plain float in
                    // arithmetic, the register allocator moves all 256 accumulators out of the
                    // AGPRs at the loop exit and spills.
                    float x;
                    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(x) : "a"(acc[i][j][v]));
                    if constexpr (decltype(scale)::value) x = __builtin_amdgcn_ldexpf(x, row_exp(i, v));
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x), rd, off, 0, decltype(cpol)::value);
                }
            }
        }
    };
    const __amdgpu_buffer_rsrc_t ry = buffer_rsrc(p.y, p.M * p.N * 4);
    const int rl = p.M - m0, cl = p.N - n0;   // valid rows / columns of this tile
    // Y is written once and not read again by this launch: non-temporal stores (measured
    // 2-3 us faster at M=2048, K=4096, where 256 whole tiles store at the end of a round).
    using y_store = std::integral_constant<int, kNonTemporal>;
    using coherent_store = std::integral_constant<int, kDeviceCoherent>;
    if (!split) {
        store_tile(ry, p.N, m0, n0, rl, cl, y_store{}, std::true_type{});
        return;
    }
    // Two halves: the first to arrive (it swaps the tile's tag from 0 to this launch's
    // epoch) writes its partial sums through to its tile's slot of the partials workspace
    // (sc1 stores) and raises the tile's flag to the epoch once those stores have
    // completed; the second (it finds its own epoch in the tag) waits for the flag, reads
    // the slot with device-coherent loads and stores its own sums plus the slot into Y,
    // once. Per split tile that moves three tiles of fp32 (slot write, slot read, Y
    // write). Y = p0 + p1 either way (fp32 addition commutes), so the result does not
    // depend on the arrival order. The second waits only for a workgroup that has already
    // arrived (and is therefore running), so the wait ends; its bound only turns a misuse
    // into an error instead of a hang. The hand-off uses no agent-scope fence (on gfx950
    // those write back or invalidate the XCD's whole L2, and an acquiring spin would
    // invalidate it on every poll). A tag that is neither 0 nor this launch's epoch means
    // another launch is using the counters (two launches on one workspace overlapping):
    // the half reports it in p.err and stores nothing, and so does a second half whose
    // flag does not come. The host turns p.err into an error status.
    int& arrival = xs[0];
    int* const cnt = p.sync + 2 * (tile - p.full);
    if (threadIdx.x == 0) {
        int seen = 0;
        if (__hip_atomic_compare_exchange_strong(cnt, &seen, p.epoch, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT))
            arrival = 0;
        else
            arrival = seen == p.epoch ? 1 : 2;
    }
    __syncthreads();
    float* const slot = p.part + (int64_t)(tile - p.full) * (BM * BN);
    const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(slot, BM * BN * 4);
    if (arrival == 0) {
        store_tile(rs, BN, 0, 0, rl, cl, coherent_store{}, std::false_type{});
        wait_vmem_order_only_release();
        __syncthreads();
        if (threadIdx.x == 0) __hip_atomic_store(cnt + 1, p.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (arrival == 2) {
        if (threadIdx.x == 0) __hip_atomic_store(p.err, kPipeErrOverlap, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        return;
    }
    int& flag_ok = xs[1];
    if (threadIdx.x == 0) {
        int ok = 0;
        for (int spin = 0; spin < p.spin_limit; ++spin) {
            if (__hip_atomic_load(cnt + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.epoch) {
                ok = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (!ok) __hip_atomic_store(p.err, kPipeErrTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        flag_ok = ok;
        // Both halves are past their use of the pair: leave it zero for the next launch.
        __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(cnt + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!flag_ok) return;
    wait_vmem_order_only_acquire();
    // Y = (acc + slot) * 2^erow, in the accumulator layout (each lane reads back the slot
    // entries the first half's lane of the same position wrote), one fragment at a time
    // with the next fragment's loads issued before this fragment's stores (the compiler
    // cannot move loads of one buffer above stores to another).
    constexpr int NF = FM * FN;
    auto frag_offset = [&](int f, int v, int ld, int rb, int cb) {   // byte offset, bit 30 set outside
        const int i = f / FN, j = f % FN;
        const int r = wm * 128 + 32 * i + 4 * lh + 8 * (v >> 2) + (v & 3), col = wn * 128 + 32 * j + lr;
        const uint32_t far = (uint32_t)(((rl - 1 - r) | (cl - 1 - col)) >> 31) & (uint32_t)kPipeFar;
        return (int)((((uint32_t)(rb + r) * (uint32_t)ld + (uint32_t)(cb + col)) * 4u) | far);
    };
    floatx16_t sv[2];
    auto load_frag = [&](int f, floatx16_t& sd) {
#pragma unroll
        for (int v = 0; v < 16; ++v)
            sd[v] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, frag_offset(f, v, BN, 0, 0), 0,
                                                                                   kDeviceCoherent));
    };
    load_frag(0, sv[0]);
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        if (f + 1 < NF) load_frag(f + 1, sv[(f + 1) & 1]);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            float a;   // an AGPR operand, as in store_tile
            asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(a) : "a"(acc[f / FN][f % FN][v]));
            const float xv = __builtin_amdgcn_ldexpf(a + sv[f & 1][v], row_exp(f / FN, v));
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, xv), ry, frag_offset(f, v, p.N, m0, n0), 0,
                                                  kNonTemporal);
        }
        __builtin_amdgcn_sched_barrier(0);   // keeps the scheduler from hoisting every load (and spilling)
    }
}

// B8: 8-bit codes (32 bytes per row and step, one zero-point byte per block); otherwise
// 4-bit codes.
template <bool B8>
__global__ __launch_bounds__(256) void mfma_w4_pipe_kernel(PipeParams p)
{
    using L = PipeLds<B8>;
    constexpr int BN = kPipeBN, FM = 4, FN = 4;
    constexpr int A_ST = L::A_ST, CG = L::CG, SG = L::SG, ZG = L::ZG;
    constexpr int OFF_A = L::OFF_A, OFF_C = L::OFF_C, OFF_S = L::OFF_S, OFF_Z = L::OFF_Z, OFF_B = L::OFF_B,
                  OFF_E = L::OFF_E;
    constexpr int B16_SZ = BN * 64;
    constexpr int CQ = B8 ? 8 : 4;   // code loads per wave and group
    extern __shared__ __attribute__((aligned(16))) uint8_t pipe_lds[];
    uint8_t* const lds = pipe_lds;
    const uint32_t lbase = lds_address(lds);

    PipeItem it;
    if (!pipe_item(p, it)) return;
    const int c0 = it.c0, nsteps = it.nsteps, m0 = it.m0, n0 = it.n0;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int wm = wave & 1, wn = wave >> 1;

    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(p.a16, p.M * p.K * 2);
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(p.b, p.N * p.row_bytes);
    const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(p.scales, p.N * p.nb * 4);
    const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(p.zp ? (const void*)p.zp : (const void*)p.scales,
                                                  p.zp ? p.N * p.zrb : 0);
    // Loop-invariant per-lane offsets; the step advance rides in the scalar soffset.
    // Codes: 4-bit, load q of a wave moves rows wave*64 + 16q .. + 15, 64 bytes each (lane
    // i: row i/4, chunk i%4); 8-bit, rows wave*64 + 8q .. + 7, 128 bytes each, lane i
    // fetching chunk (i%8) ^ (row%8) of row i/8 into slot i%8 (so that the dequant's
    // 32-byte reads of 8 consecutive rows hit distinct banks).
    int avo[4], cvo[CQ];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int r = wave * 64 + 16 * q + (lane >> 2);
        const int m = m0 + r;
        avo[q] = m < p.M ? m * p.K * 2 + c0 * 64 + pipe_slot(r, lane & 3) * 16 : kPipeFar;
    }
#pragma unroll
    for (int q = 0; q < CQ; ++q) {
        if constexpr (B8) {
            const int r = wave * 64 + 8 * q + (lane >> 3), n = n0 + r;
            cvo[q] = n < p.N ? n * p.row_bytes + c0 * 32 + (((lane & 7) ^ (r & 7)) * 16) : kPipeFar;
        } else {
            const int n = n0 + wave * 64 + 16 * q + (lane >> 2);
            cvo[q] = n < p.N ? n * p.row_bytes + c0 * 16 + (lane & 3) * 16 : kPipeFar;
        }
    }
    const int brow = wave * 64 + lane;   // the weight row this lane loads scales for and dequantizes
    const int bn = n0 + brow;
    const int svo = bn < p.N ? bn * p.nb * 4 + c0 * 4 : kPipeFar;
    const int zvo = bn < p.N ? bn * p.zrb + (B8 ? c0 : c0 / 2) : kPipeFar;
    // Without zero points the zero-point loads read 0 (an empty buffer) and zadd is the
    // operator's default, 2^(bits - 1).
    const uint32_t zadd = p.zp ? 0u : (B8 ? 128u : 8u);
    const int last = nsteps - 1;

    auto issue_a = [&](int t, int st) {   // step t -> stage st (clamped: a prefetch past the end re-reads)
        const int tc = min(t, last);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            lds_load16(ra, avo[q], tc * 64, lbase + OFF_A + st * A_ST + (wave * 64 + 16 * q) * 64);
    };
    auto issue_b = [&](int g, int buf) {  // steps 4g .. 4g+3 -> buffer buf (CQ + 2 loads)
        const int gc = min(g, last >> 2);
#pragma unroll
        for (int q = 0; q < CQ; ++q)
            lds_load16(rb, cvo[q], gc * L::CROW, lbase + OFF_C + buf * CG + (wave * 64 + (64 / CQ) * q) * L::CROW);
        lds_load16(rsc, svo, gc * 16, lbase + OFF_S + buf * SG + wave * 64 * 16);
        if constexpr (B8)
            lds_load4(rz, zvo, gc * 4, lbase + OFF_Z + buf * ZG + wave * 64 * 4);
        else
            lds_load2(rz, zvo, gc * 2, lbase + OFF_Z + buf * ZG + wave * 64 * 4);
    };
    struct Raw {
        u32x4_t q[B8 ? 2 : 1];
        float s;
        uint32_t zb;
    };
    auto read_raw = [&](int t, int buf) {
        Raw r;
        const int ph = t & 3;
        if constexpr (B8) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
                r.q[h] = *reinterpret_cast<const u32x4_t*>(lds + OFF_C + buf * CG + brow * 128 +
                                                           (((2 * ph + h) ^ (brow & 7)) * 16));
        } else {
            r.q[0] = *reinterpret_cast<const u32x4_t*>(lds + OFF_C + buf * CG + brow * 64 + ph * 16);
        }
        r.s = *reinterpret_cast<const float*>(lds + OFF_S + buf * SG + brow * 16 + ph * 4);
        r.zb = *reinterpret_cast<const uint32_t*>(lds + OFF_Z + buf * ZG + brow * 4);
        return r;
    };
    auto dequant = [&](const Raw& raw, int t) {
        const uint32_t zp = B8 ? ((raw.zb >> ((t & 3) * 8)) & 0xFFu) + zadd : ((raw.zb >> ((t & 3) * 4)) & 0x0Fu) + zadd;
        const h2_t zb = as_h2(kHalfMagic | (zp << 16) | zp);
        const _Float16 sh = (_Float16)raw.s;
        const h2_t s2 = h2_t{sh, sh};
        uint8_t* dst = lds + OFF_B + (t & 1) * B16_SZ + brow * 64;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t o[4];
            if constexpr (B8) {
                const u32x4_t& c = raw.q[j >> 1];
                dequant8_f16_b8((j & 1) ? c.z : c.x, (j & 1) ? c.w : c.y, zb, s2, o);
            } else {
                const u32x4_t& c = raw.q[0];
                dequant8_f16(j == 0 ? c.x : j == 1 ? c.y : j == 2 ? c.z : c.w, zb, s2, o);
            }
            *reinterpret_cast<u32x4_t*>(dst + pipe_slot(brow, j) * 16) = u32x4_t{o[0], o[1], o[2], o[3]};
        }
    };

    floatx16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = floatx16_t{};
    }
    const int lr = lane & 31, lh = lane >> 5;
    // MFMA operands of one half step (16 k): 4 A and 4 B fragments.
    struct Ops {
        half8_t a[FM], b[FN];
    };
    auto load_ops = [&](int st, int bbuf, int sub, Ops& o) {
        const uint8_t* As = lds + OFF_A + st * A_ST;
        const uint8_t* Bs = lds + OFF_B + bbuf * B16_SZ;
        const int j = 2 * sub + lh;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int r = wm * 128 + 32 * i + lr;
            o.a[i] = *reinterpret_cast<const half8_t*>(As + r * 64 + pipe_slot(r, j) * 16);
        }
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const int r = wn * 128 + 32 * i + lr;
            o.b[i] = *reinterpret_cast<const half8_t*>(Bs + r * 64 + pipe_slot(r, j) * 16);
        }
    };
    auto mfma_ops = [&](const Ops& o) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int jn = 0; jn < FN; ++jn)
                acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(o.a[i], o.b[jn], acc[i][jn], 0, 0, 0);
        }
    };

    // Step t (A stage t % NA, fp16 weight tile t & 1), with R0 holding the operands of its
    // first half (k 0-15):
    //   first half:  read R1 (k 16-31) and the raw weights of step t+2; MFMAs on R0,
    //                interleaved with the dequant of step t+1 into tile (t+1) & 1;
    //                wait for A(t+1); barrier;
    //   second half: read R0 of step t+1; MFMAs on R1, interleaved with the issue of the
    //                next loads.
    // So every LDS read runs under MFMAs that do not depend on it. Each wait is a vmcnt
    // count of the loads issued after the one waited for:
    //   4-bit: A issued 3 steps ahead into 4 stages; weight group g lives in raw buffer
    //   g % 3 and is issued two groups (8 steps) ahead, at t % 4 == 0 after A(t+3). Issue
    //   order per wave: B(0) B(1) A(0) A(1) A(2), then per step A(t+3) [4 loads] and, at
    //   t % 4 == 0, B(t/4+2) [6 loads].
    //   8-bit: A issued 2 steps ahead into 3 stages; group g lives in raw buffer g % 2 and
    //   is issued at t % 4 == 1 of group g - 2, after A(t+2), once the last raw reads of
    //   group g - 2 (at step 4g - 7) are behind the step's barrier. Issue order: B(0) B(1)
    //   A(0) A(1), then per step A(t+2) [4] and, at t % 4 == 1, B(t/4+2) [10].
    Ops R0, R1;
    // The tile's row exponents go straight to LDS (row t at OFF_E + 4t), oldest of all the
    // loads, so every wait below covers them too; rows past M read zero.
    {
        const int r = m0 + wave * 64 + lane;
        lds_load4(buffer_rsrc(p.rexp, p.M * 4), r < p.M ? r * 4 : kPipeFar, 0, lbase + OFF_E + wave * 256);
    }
    issue_b(0, 0);
    issue_b(1, 1);
    issue_a(0, 0);
    issue_a(1, 1);
    if constexpr (!B8) {
        issue_a(2, 2);
        wait_vmcnt<8>();                     // B(0), B(1), A(0): then A(1), A(2)
    } else {
        wait_vmcnt<4>();                     // B(0), B(1), A(0): then A(1)
    }
    Raw raw = read_raw(0, 0);
    dequant(raw, 0);
    raw = read_raw(1, 0);
    lds_barrier();
    load_ops(0, 0, 0, R0);
    // st: A stage of step t; rbuf: raw buffer of step t+2; nbuf: the buffer of the weight
    // group this step issues (if any).
    auto step = [&](int t, auto phase, auto wait, int st, int rbuf, int nbuf) {
        constexpr int ph = decltype(phase)::value;
        __builtin_amdgcn_sched_barrier(0);
        load_ops(st, ph & 1, 1, R1);
        Raw rn = read_raw(t + 2, rbuf);
        mfma_ops(R0);
        dequant(raw, t + 1);
        // 16 MFMAs, each followed by one LDS operation (the reads, then the dequant's 4
        // writes) and a share of the dequant's VALU work: about 5 VALU instructions fit
        // in the shadow of one 32-cycle MFMA.
        constexpr int NR = B8 ? 12 : 11;
#pragma unroll
        for (int g = 0; g < NR; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
        }
        if constexpr (!B8) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_barrier(0);
        raw = rn;
        wait_vmcnt<decltype(wait)::value>();
        lds_barrier();
        if constexpr (B8) {
            const int st1 = st == 2 ? 0 : st + 1;
            load_ops(st1, (ph + 1) & 1, 0, R0);
            mfma_ops(R1);
            issue_a(t + 2, st1 == 2 ? 0 : st1 + 1);
            if constexpr (ph == 1) issue_b((t >> 2) + 2, nbuf);
        } else {
            load_ops((ph + 1) & 3, (ph + 1) & 1, 0, R0);
            mfma_ops(R1);
            issue_a(t + 3, (ph + 3) & 3);
            if constexpr (ph == 0) issue_b((t >> 2) + 2, nbuf);
        }
        // The second half is left to the compiler's scheduler: a pattern of one MFMA per LDS
        // read (8 reads, then 8 MFMAs) measured 0.2-0.5% slower (M=2048 K=11008 214.8 against
        // 213.8 us; K=4096 201.3 against 201.0 us).
        __builtin_amdgcn_sched_barrier(0);
    };
    using std::integral_constant;
    if constexpr (B8) {
        int b0 = 0, b1 = 1;                // raw buffers of groups g, g+1
        int st = 0;                        // A stage of step t
        for (int t = 0; t < nsteps; t += 4) {
            const int s1 = st == 2 ? 0 : st + 1, s2 = s1 == 2 ? 0 : s1 + 1;
            step(t, integral_constant<int, 0>{}, integral_constant<int, 0>{}, st, b0, b0);        // A(t+1): last issued
            step(t + 1, integral_constant<int, 1>{}, integral_constant<int, 0>{}, s1, b0, b0);    // A(t+2): last issued
            step(t + 2, integral_constant<int, 2>{}, integral_constant<int, 10>{}, s2, b1, b0);   // A(t+3): then B(g+2)
            step(t + 3, integral_constant<int, 3>{}, integral_constant<int, 0>{}, st, b1, b0);    // A(t+4): last issued
            st = s1;                        // (t + 4) % 3
            const int bt = b0;
            b0 = b1;
            b1 = bt;
        }
    } else {
        int b0 = 0, b1 = 1, b2 = 2;           // raw buffers of groups g, g+1, g+2
        for (int t = 0; t < nsteps; t += 4) {
            step(t, integral_constant<int, 0>{}, integral_constant<int, 4>{}, 0, b0, b2);       // A(t+1): then A(t+2)
            step(t + 1, integral_constant<int, 1>{}, integral_constant<int, 10>{}, 1, b0, b2);  // A(t+2): then A(t+3), B(g+2)
            step(t + 2, integral_constant<int, 2>{}, integral_constant<int, 10>{}, 2, b1, b2);  // A(t+3): then B(g+2), A(t+4)
            step(t + 3, integral_constant<int, 3>{}, integral_constant<int, 4>{}, 3, b1, b2);   // A(t+4): then A(t+5)
            const int bt = b0;
            b0 = b1;
            b1 = b2;
            b2 = bt;
        }
    }
    wait_vmcnt<0>();
    __syncthreads();   // every wave is past its last LDS access of the main loop; exponents landed

    pipe_epilogue(p, it, acc, reinterpret_cast<const int*>(lds + OFF_E), reinterpret_cast<int*>(lds + OFF_A));
}

}  // namespace msnb
