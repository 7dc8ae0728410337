// mfma_w4_rb.h — 4- and 8-bit MatMulNBits prefill GEMM with the weights dequantized
// straight into MFMA operand registers (M > 16, block sizes 32..., K a multiple of 128).
//
// Y[M,N] = A[M,K] * W[N,K]^T, W = fl16((q - zp) * fl16(s)), A the fp16 copy made by
// a_rows_f16_kernel (row m scaled by 2^-rexp[m]; each 8-k group in the order
// k0,k4,k1,k5,k2,k6,k3,k7, the order in which one dword of packed codes dequantizes).
//
// A workgroup (4 waves) computes a 128 x (64 NF) tile of Y over a range of 128-k blocks
// (NF = 1, 2 or 4: narrower tiles let launches with few rows of A fill the CUs with a
// smaller K split):
//   * wave w owns weight rows n0 + 16 NF w .. (NF fragments of 16) and all 128 rows of
//     A (8 fragments of 16): 8 NF v_mfma_f32_16x16x32_f16 per 32-k step, 32 NF fp32
//     accumulators per lane. Every dequantized weight feeds 128 rows of A, so the
//     dequant's VALU work (15 instructions per dword of 8 codes) is about half the MFMA
//     time. (Two waves per SIMD at 64 x 64 each, which both dequantize the same rows,
//     measured slower: their dequant alone matches the MFMA time.)
//   * weights never touch LDS: lane (n = lane % 16, s = lane / 16) loads the 16-byte chunk
//     s of its row's 64-byte block of codes (plus the chunk's scale and zero point) into a
//     ring of registers three blocks deep, and dword j of the chunk becomes the B operand
//     of step j (k = 32 s + 8 j + [0, 8)). With 8-bit codes (B8) a row's block is 128
//     bytes: the lane loads its 32 codes as two chunks, and dwords 2j, 2j + 1 make step j
//     (dequant8_f16_b8, the same pair order and rounding);
//   * the scales and zero points come from the handle's chunk-major copy (rb_chunk_layout
//     _kernel, built once): one dword per (128-k block g, row n, chunk c) at (g N + n) 4 + c
//     holding fl16(s) in its low half and the fp16 1024 + zp in its high half (the two
//     constants of the dequant, exact), so a fragment's 16 rows read 256 contiguous bytes
//     per block (from the operator's [N][nb] layout they touched 16 lines each; that cost
//     2-23 us of 43-127 us on the 7B prefill shapes);
//   * A goes through LDS, double-buffered, one block (128 rows x 128 k, 32 KB) per buffer,
//     laid out so that the A operand of (step j, fragment f) is 1 KB read by the 64 lanes
//     in order (no bank conflicts). The next block's A is loaded into registers while the
//     current block computes, written to the other buffer at the start of the next block;
//     one barrier per block.
//   * K split (ksw > 1, for launches with too few tiles to fill the CUs): workgroup kw of
//     a tile writes its partial sums to slice kw of a [ksw][M][N] workspace with plain
//     stores, and rb_reduce_kernel adds the slices in index order into Y afterwards
//     (deterministic; the kernel boundary orders the two launches). The reduce also
//     multiplies row m by 2^rexp[m] (exact), so it runs for ksw = 1 too: scaling the
//     accumulators in this kernel's epilogue moved them out of the AGPRs at the loop exit
//     (hundreds of spilled registers).
// Rows past M and columns past N read zeros (out-of-range buffer offsets) and are not
// stored.
#pragma once
#include "mfma_w4_pipe.h"

namespace msnb {

constexpr int kRbBM = 128;   // rows of A per tile; the tile's columns are 64 * NF (NF = 1, 2, 4)
constexpr int kRbRing = 3;                     // weight blocks in registers
constexpr int kRbBufBytes = kRbBM * 128 * 2;   // one block of fp16 A

struct RbParams {
    const uint8_t* b;          // [N][row_bytes]
    const uint32_t* sz4;       // [K / 128][N][4] fl16(s) | fp16(1024 + zp) << 16 of each 32-code chunk
    const _Float16* a16;       // [M][K] fp16, permuted within 8-k groups, row m scaled by 2^-rexp[m]
    float* out;                // the workspace: ksw slices of `slice` floats
    int64_t slice;             // M * N rounded up to a multiple of 4 (16-byte aligned slices)
    int row_bytes, M, N, K;
    int tiles_m, tiles_n, ksw;
};

template <int NF, bool B8>
__global__ __launch_bounds__(256) void mfma_w4_rb_kernel(RbParams p)
{
    constexpr int CW = B8 ? 2 : 1;       // 16-byte code chunks per lane and 128-k block
    constexpr int BLK = 64 * CW;         // code bytes per row and 128-k block
    constexpr int MF = kRbBM / 16, BN = 64 * NF;
    __shared__ __attribute__((aligned(16))) uint8_t lds_a[2 * kRbBufBytes];

    const int items = p.tiles_m * p.tiles_n * p.ksw;
    // Consecutive items share (m tile, K range), so an XCD's range reuses its A in L2.
    const int item = xcd_tile(blockIdx.x, items);
    if (item >= items) return;
    const int nt = item % p.tiles_n, rest = item / p.tiles_n;
    const int kw = rest % p.ksw, mt = rest / p.ksw;
    const int G = p.K >> 7;
    const int g0 = (int)((int64_t)kw * G / p.ksw), cnt = (int)((int64_t)(kw + 1) * G / p.ksw) - g0;
    const int m0 = mt * kRbBM, n0 = nt * BN;

    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int ln = lane & 15, ls = lane >> 4;

    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(p.a16, p.M * p.K * 2);
    const __amdgpu_buffer_rsrc_t rb_ = buffer_rsrc(p.b, p.N * p.row_bytes);
    const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(p.sz4, G * p.N * 16);

    // ---- A staging: thread t moves chunks q = t + 256 u (u = 0..7) of a block; chunk q is
    // (step j = q >> 9, fragment f = (q >> 6) & 7, s = (q >> 4) & 3, row r = q & 15) and
    // holds A[m0 + 16 f + r][128 g + 32 s + 8 j ...] (16 bytes). ----
    int aoff[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int q = tid + 256 * u;
        const int j = q >> 9, f = (q >> 6) & 7, s = (q >> 4) & 3, r = q & 15;
        const int m = m0 + 16 * f + r;
        aoff[u] = m < p.M ? (m * p.K + 32 * s + 8 * j) * 2 : kOOB;
    }
    u32x4_t areg[8];
    auto load_a = [&](int i) {   // block g0 + i -> registers (zeros past the range)
        const bool ok = i < cnt;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            areg[u] = __builtin_amdgcn_raw_buffer_load_b128(ra, ok && aoff[u] != kOOB ? aoff[u] + (g0 + i) * 256 : kOOB, 0, 0);
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
            *reinterpret_cast<u32x4_t*>(&lds_a[buf * kRbBufBytes + (tid + 256 * u) * 16]) = areg[u];
    };

    // ---- weights: lane (ln, ls) of fragment f is row n0 + 64 wave + 16 f + ln ----
    int cb[NF], sb[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        const int n = n0 + 16 * NF * wave + 16 * f + ln;
        const bool in = n < p.N;
        cb[f] = in ? n * p.row_bytes + ls * 16 * CW : kOOB;
        sb[f] = in ? n * 16 + ls * 4 : kOOB;
    }
    struct WBlk {
        u32x4_t c[NF][CW];
        uint32_t sz[NF];
    };
    WBlk w[kRbRing];
    auto load_w = [&](WBlk& wb, int i) {
        const bool ok = i < cnt;
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const bool okf = ok && cb[f] != kOOB;
#pragma unroll
            for (int h = 0; h < CW; ++h)
                wb.c[f][h] = __builtin_amdgcn_raw_buffer_load_b128(rb_, okf ? cb[f] + (g0 + i) * BLK + 16 * h : kOOB, 0, 0);
            wb.sz[f] = __builtin_amdgcn_raw_buffer_load_b32(rsc, okf ? sb[f] + (g0 + i) * p.N * 16 : kOOB, 0, 0);
        }
    };

    floatx4_t acc[MF][NF];
#pragma unroll
    for (int f = 0; f < MF; ++f) {
#pragma unroll
        for (int e = 0; e < NF; ++e) acc[f][e] = floatx4_t{};
    }

    // Per-block dequant constants of ring slot wb (block g0 + i): (1024 + zp) and fl16(s),
    // both twice, per fragment (one v_perm each from the packed dword).
    auto prep = [&](const WBlk& wb, int i, uint32_t (&zz)[NF], h2_t (&s2)[NF]) {
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            zz[f] = __builtin_amdgcn_perm(wb.sz[f], wb.sz[f], 0x03020302u);
            s2[f] = as_h2(__builtin_amdgcn_perm(wb.sz[f], wb.sz[f], 0x01000100u));
        }
    };
    // A operand of (step j, fragment mf): 1 KB, lane-ordered.
    auto read_a1 = [&](int buf, int j, int mf) {
        return *reinterpret_cast<const half8_t*>(&lds_a[buf * kRbBufBytes + ((j * MF + mf) * 64 + lane) * 16]);
    };
    // B operands of step j, fragment f only.
    auto deq1 = [&](const WBlk& wb, int j, int f, uint32_t zzf, h2_t s2f) {
        uint32_t o[4];
        if constexpr (B8) {
            // step j: codes 8j .. 8j + 7 of the lane's 32, dwords 2j (k0..k3) and 2j + 1 (k4..k7)
            const u32x4_t& cw = wb.c[f][j >> 1];
            const uint32_t d0 = (j & 1) ? cw.z : cw.x, d1 = (j & 1) ? cw.w : cw.y;
            dequant8_f16_b8(d0, d1, as_h2(zzf), s2f, o);
        } else {
            const u32x4_t& cw = wb.c[f][0];
            const uint32_t x = j == 0 ? cw.x : j == 1 ? cw.y : j == 2 ? cw.z : cw.w;
            dequant8_f16(x, as_h2(zzf), s2f, o);
        }
        return __builtin_bit_cast(half8_t, u32x4_t{o[0], o[1], o[2], o[3]});
    };

    // ---- prologue, in the steady state's issue order: A(0) W(0) W(1) | A(1) W(2) ----
    load_a(0);
    __builtin_amdgcn_sched_barrier(0);
    load_w(w[0], 0);
    __builtin_amdgcn_sched_barrier(0);
    load_w(w[1], 1);
    __builtin_amdgcn_sched_barrier(0);
    store_a(0);
    load_a(1);
    __builtin_amdgcn_sched_barrier(0);
    load_w(w[2], 2);
    __builtin_amdgcn_sched_barrier(0);
    half8_t bq0[NF];   // B operands of step 0 of the next block, prepared under the last step's MFMAs
    {
        uint32_t zz[NF];
        h2_t s2[NF];
        prep(w[0], 0, zz, s2);
#pragma unroll
        for (int f = 0; f < NF; ++f) bq0[f] = deq1(w[0], 0, f, zz[f], s2[f]);
    }
    __syncthreads();

    // ---- main loop ----
    // Block i: (A(i+1) registers -> LDS; issue A(i+2)); 32 groups (step j, fragment mf) of
    // NF MFMAs, in chunks of RC groups: the A operands of a chunk (RC fragments of 1 KB,
    // lane-ordered) are read from LDS in one burst while the previous chunk computes, and
    // the B operands of step j + 1 are dequantized one fragment per group under the first
    // NF groups of step j (the last step prepares step 0 of block i+1 from the next ring
    // slot); then W(i+3) goes into the slot just used, which becomes the ring's last;
    // barrier. At the top of block i the outstanding loads are A(i+1) then W(i+2), so the A
    // store waits for A(i+1) alone. RC = 8 (a whole step) where the registers allow, 4 at
    // NF = 4. The loop body carries no scheduling pins: with `sched_barrier` between the
    // bursts and a `sched_group_barrier` pattern of 1 MFMA then 4 VALU, the register
    // allocator kept 14 of the 32 accumulator fragments at NF = 4 in other AGPRs across the
    // back edge (112 AGPR<->VGPR moves per block, 76 s_nop); the compiler's own schedule has
    // none (443 VALU-side instructions and 21 s_nop per block) and measured faster at every
    // NF (7B gate, M = 17 / 64: 40.0 / 44.2 -> 34.8 / 39.1 us; M=128, K=4096: 41.6 -> 38.3 us;
    // M=512, K=11008: 81.4 -> 73.6 us; NF = 2 at M=128, K=11008: 35.5 -> 34.9 us).
    constexpr int RC = NF == 4 ? 4 : 8, NCH = 4 * MF / RC;
    auto body = [&](int i, WBlk& wb, const WBlk& wbn) {
        const int buf = i & 1;
        half8_t aw[2][RC];
#pragma unroll
        for (int r = 0; r < RC; ++r) aw[0][r] = read_a1(buf, r / MF, r % MF);
        if (i + 1 < cnt) store_a((i + 1) & 1);
        load_a(i + 2);
        uint32_t zz[NF], zzn[NF];
        h2_t s2[NF], s2n[NF];
        prep(wb, i, zz, s2);
        prep(wbn, i + 1, zzn, s2n);
        half8_t bq[NF], bqn[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f) bq[f] = bq0[f];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            if (c + 1 < NCH) {
#pragma unroll
                for (int r = 0; r < RC; ++r) {
                    const int t = (c + 1) * RC + r;
                    aw[(c + 1) & 1][r] = read_a1(buf, t / MF, t % MF);
                }
            }
#pragma unroll
            for (int r = 0; r < RC; ++r) {
                const int t = c * RC + r, j = t / MF, mf = t % MF;
#pragma unroll
                for (int f = 0; f < NF; ++f)
                    acc[mf][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw[c & 1][r], bq[f], acc[mf][f], 0, 0, 0);
                if (mf < NF) bqn[mf] = j < 3 ? deq1(wb, j + 1, mf, zz[mf], s2[mf]) : deq1(wbn, 0, mf, zzn[mf], s2n[mf]);
                if (mf == MF - 1) {
#pragma unroll
                    for (int f = 0; f < NF; ++f) bq[f] = bqn[f];
                }
            }
        }
#pragma unroll
        for (int f = 0; f < NF; ++f) bq0[f] = bq[f];
        load_w(wb, i + kRbRing);
        __syncthreads();
    };
    // One body per iteration and the ring rotated by value (a few register moves per
    // block): with the body unrolled once per ring slot, three exits and three register
    // sets per slot, the register allocator moved every accumulator through VGPRs around
    // its MFMAs (four v_accvgpr_write per MFMA at NF = 4).
    for (int i = 0; i < cnt; ++i) {
        body(i, w[0], w[1]);
        const WBlk t0 = w[0];
        w[0] = w[1];
        w[1] = w[2];
        w[2] = t0;
    }

    // ---- epilogue: acc[mf][f][v] is out[m0 + 16 mf + 4 ls + v][n0 + 16 NF wave + 16 f + ln] ----
    float* const out = p.out + kw * p.slice;
    const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(out, p.M * p.N * 4);
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        const int n = n0 + 16 * NF * wave + 16 * f + ln;
#pragma unroll
        for (int mf = 0; mf < MF; ++mf) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int m = m0 + 16 * mf + 4 * ls + v;
                const float x = acc[mf][f][v];   // a scalar first: a bit cast of a vector element reads element 0
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x), ro,
                                                      m < p.M && n < p.N ? (m * p.N + n) * 4 : kOOB, 0, 0);
            }
        }
    }
}

// y[e] = 2^rexp[e / N] * (sum over kw of slice kw at e, in kw order) for e < n (< 2^31);
// the slices are slice4 float4 groups apart (16-byte aligned), y only 4-byte aligned.
// Y = 2^rexp[m] * sum over the ksw slices, in slice order (deterministic); thread i
// takes elements 4i .. 4i + 3 with up to kRbRedBatch slices' loads in flight at once.
// Bound by the slices' bytes: (ksw + 1) * 4 M N (28 MB in 7.8 us at M = 128, N = 11008,
// ksw = 4).
constexpr int kRbRedBatch = 16;
// With vec set (N % 4 == 0 and y 16-byte aligned) the four elements of thread i lie in one
// row and go out as one 16-byte store.
__global__ __launch_bounds__(256) void rb_reduce_kernel(const float4* __restrict__ part, float* __restrict__ y,
                                                        const int* __restrict__ rexp, int n, int N, int slice4, int ksw,
                                                        int vec)
{
    const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(part, ksw * slice4 * 16);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < slice4; i += gridDim.x * blockDim.x) {
        float4 t;
        for (int w0 = 0; w0 < ksw; w0 += kRbRedBatch) {
            u32x4_t v[kRbRedBatch];
#pragma unroll
            for (int u = 0; u < kRbRedBatch; ++u)
                v[u] = __builtin_amdgcn_raw_buffer_load_b128(rp, w0 + u < ksw ? ((w0 + u) * slice4 + i) * 16 : kOOB, 0, 0);
#pragma unroll
            for (int u = 0; u < kRbRedBatch; ++u) {
                const float4 f = __builtin_bit_cast(float4, v[u]);
                if (w0 + u == 0) {
                    t = f;
                } else if (w0 + u < ksw) {
                    t.x += f.x;
                    t.y += f.y;
                    t.z += f.z;
                    t.w += f.w;
                }
            }
        }
        if (vec) {
            const int e = rexp[(4 * i) / N];
            const float4 o = {__builtin_amdgcn_ldexpf(t.x, e), __builtin_amdgcn_ldexpf(t.y, e),
                              __builtin_amdgcn_ldexpf(t.z, e), __builtin_amdgcn_ldexpf(t.w, e)};
            *reinterpret_cast<float4*>(y + 4 * i) = o;
            continue;
        }
        const float tv[4] = {t.x, t.y, t.z, t.w};
        int m = (4 * i) / N, col = 4 * i - m * N;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if (4 * i + c < n) y[4 * i + c] = __builtin_amdgcn_ldexpf(tv[c], rexp[m]);
            if (++col == N) {
                col = 0;
                ++m;
            }
        }
    }
}

// The chunk-major copy of a handle's scales and zero points that mfma_w4_rb reads: entry
// (g, n, c) packs fl16 of the scale and 1024 + the zero point (2^(bits-1) without zero
// points) of the quantization block that holds codes 128 g + 32 c .. + 31 of row n.
__global__ __launch_bounds__(256) void rb_chunk_layout_kernel(const float* __restrict__ scales,
                                                              const uint8_t* __restrict__ zp,
                                                              uint32_t* __restrict__ sz4, int N, int G, int nb,
                                                              int zrb, int log2bs, int bits)
{
    const int64_t total = (int64_t)G * N * 4;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
        const int c = (int)(e & 3);
        const int64_t gn = e >> 2;
        const int g = (int)(gn / N), n = (int)(gn - (int64_t)g * N);
        const int blk = (g * 128 + 32 * c) >> log2bs;
        uint32_t z;
        if (bits == 8)
            z = zp ? zp[(int64_t)n * zrb + blk] : 128u;
        else
            z = zp ? (zp[(int64_t)n * zrb + (blk >> 1)] >> ((blk & 1) * 4)) & 0x0Fu : 8u;
        // fl16(s) (round to nearest even, the dequant's rounding of the scale) and the fp16
        // 1024 + zp (exact for zp < 1024)
        const _Float16 sh = (_Float16)scales[(int64_t)n * nb + blk];
        sz4[e] = (uint32_t)__builtin_bit_cast(uint16_t, sh) | ((0x6400u | z) << 16);
    }
}

}  // namespace msnb
