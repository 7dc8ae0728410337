// mfma_w4_preg.h — the pipelined INT4 prefill GEMM (mfma_w4_pipe.h) with the weights
// dequantized by each wave straight into its MFMA B-operand registers.
//
// Same tile (256x256 per workgroup, 4 waves in 2x2, each 128x128 as 4x4
// v_mfma_f32_32x32x16_f16 fragments in AGPRs), the same buffer->LDS load pipeline
// (A 4 stages issued 3 steps ahead; codes, scales and zero points per group of 4 steps in
// three buffers issued two groups ahead), the same waits, K split and epilogue.
//
// What changes is where the weights are dequantized. mfma_w4_pipe has every lane
// dequantize one weight row into an fp16 tile in LDS, which the two waves of a column
// half then read as B operands: per step and CU that is 16 KB of LDS writes and 32 KB of
// reads, about half of the step's LDS traffic. Here each wave reads the raw codes of its
// own 128 weight rows from LDS (2 KB per step instead of 8 KB of fp16) and dequantizes
// them in registers, with the same packed-half arithmetic
// (W = fl16((q - zp) * fl16(s))). The two waves of a column half both dequantize the
// same rows, so the VALU work per wave doubles (about 4 VALU instructions per MFMA), in
// exchange for a step's LDS traffic dropping from about 107 KB to about 66 KB per CU.
//
// k order. The B operand of a 32x32x16 MFMA holds, in lane (n = lane % 32, h = lane / 32),
// 8 consecutive-in-operand k of column n. One dword of codes (8 codes) dequantizes to
// exactly one such operand, so a lane's operands are whole dwords of its row. Within a
// group of 4 steps (128 k = 16 dwords of codes per row, dword d = codes 8d .. 8d+7),
// step ph, lane half h and MFMA sub-step s use dword
//     d = 4 * (2 * (ph >> 1) + h) + 2 * (ph & 1) + s,
// so that one 16-byte read per lane and fragment (chunk 2 * (ph >> 1) + h of the row's
// group) serves two steps. With block size 32 that chunk is one quantization block, so a
// lane's scale and zero point change every second step, and a step covers half of two
// blocks. A's LDS stage of step ph holds, at logical chunk j = 2h + s,
// A's 8-k chunk d of the group: both operands carry the same k, so the dot product is
// unchanged (its terms are only summed in another order).
//
// Code chunks are stored XOR-swizzled per row (chunk c of row r at slot c ^ ((r >> 2) & 3))
// so that a wave's 16-byte reads of 16 consecutive rows cover 16 distinct bank groups.
#pragma once
#include "mfma_w4_pipe.h"

namespace msnb {

constexpr int kPregLdsBytes = 4 * kPipeBM * 64 + 3 * (kPipeBN * 64 + kPipeBN * 16 + kPipeBN * 4);

// 16-byte A chunk (of 16 per row and group) that logical chunk j of step t's stage holds:
// preg_step_chunk(t) + preg_lane_chunk(j).
__device__ __forceinline__ int preg_step_chunk(int t) { return 8 * ((t >> 1) & 1) + 2 * (t & 1); }
__device__ __forceinline__ int preg_lane_chunk(int j) { return 4 * (j >> 1) + (j & 1); }
// LDS slot of code chunk c (0..3) of tile row r, and the chunk slot c holds (an involution).
__device__ __forceinline__ int preg_code_slot(int r, int c) { return c ^ ((r >> 2) & 3); }

__global__ __launch_bounds__(256) void mfma_w4_preg_kernel(PipeParams p)
{
    constexpr int BM = kPipeBM, BN = kPipeBN, FM = 4, FN = 4;
    constexpr int A_ST = BM * 64;                               // one step of A
    constexpr int CG = BN * 64, SG = BN * 16, ZG = BN * 4;      // one group: codes, scales, zp
    constexpr int OFF_A = 0, OFF_C = OFF_A + 4 * A_ST, OFF_S = OFF_C + 3 * CG, OFF_Z = OFF_S + 3 * SG;
    extern __shared__ __attribute__((aligned(16))) uint8_t preg_lds[];
    uint8_t* const lds = preg_lds;
    const uint32_t lbase = lds_address(lds);

    PipeItem it;
    if (!pipe_item(p, it)) return;
    const int c0 = it.c0, nsteps = it.nsteps, m0 = it.m0, n0 = it.n0;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int wm = wave & 1, wn = wave >> 1;
    const int lr = lane & 31, lh = lane >> 5;

    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(p.a16, p.M * p.K * 2);
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(p.b, p.N * p.row_bytes);
    const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(p.scales, p.N * p.nb * 4);
    const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(p.zp ? (const void*)p.zp : (const void*)p.scales,
                                                  p.zp ? p.N * p.zrb : 0);
    // Loop-invariant per-lane offsets; the step advance rides in the scalar soffset. The
    // lane filling LDS slot (r, lane & 3) loads the chunk that slot holds.
    int avo[4], cvo[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int r = wave * 64 + 16 * q + (lane >> 2);
        const int m = m0 + r;
        avo[q] = m < p.M ? m * p.K * 2 + c0 * 64 + preg_lane_chunk(pipe_slot(r, lane & 3)) * 16 : kPipeFar;
        const int n = n0 + r;
        cvo[q] = n < p.N ? n * p.row_bytes + c0 * 16 + preg_code_slot(r, lane & 3) * 16 : kPipeFar;
    }
    const int brow = wave * 64 + lane;   // the weight row this lane loads scales and zero points for
    const int bn = n0 + brow;
    const int svo = bn < p.N ? bn * p.nb * 4 + c0 * 4 : kPipeFar;
    const int zvo = bn < p.N ? bn * p.zrb + c0 / 2 : kPipeFar;
    const int last = nsteps - 1;

    auto issue_a = [&](int t, int st) {   // step t -> stage st (clamped: a prefetch past the end re-reads)
        const int tc = min(t, last);
        const int soff = (tc >> 2) * 256 + preg_step_chunk(tc) * 16;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            lds_load16(ra, avo[q], soff, lbase + OFF_A + st * A_ST + (wave * 64 + 16 * q) * 64);
    };
    auto issue_b = [&](int g, int buf) {  // steps 4g .. 4g+3 -> buffer buf
        const int gc = min(g, last >> 2);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            lds_load16(rb, cvo[q], gc * 64, lbase + OFF_C + buf * CG + (wave * 64 + 16 * q) * 64);
        lds_load16(rsc, svo, gc * 16, lbase + OFF_S + buf * SG + wave * 64 * 16);
        lds_load2(rz, zvo, gc * 2, lbase + OFF_Z + buf * ZG + wave * 64 * 4);
    };

    // Code chunk (2 * pp + lh) of the four fragment rows of this lane, group buffer buf.
    auto read_codes = [&](int buf, int pp, u32x4_t (&rc)[FN]) {
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const int rr = wn * 128 + 32 * i + lr;
            rc[i] = *reinterpret_cast<const u32x4_t*>(lds + OFF_C + buf * CG + rr * 64 +
                                                      preg_code_slot(rr, 2 * pp + lh) * 16);
        }
    };
    // Block size 32: chunk c of a row's group is block c of the group, so lane half lh
    // needs blocks lh (steps 0-1) and 2 + lh (steps 2-3). Their fp16 scales and zero
    // points, as the packed pairs the dequant subtracts and multiplies by, are formed once
    // per group: S2[i][p] = (s, s) and ZB[i][p] = (1024 + zp, 1024 + zp) of block 2p + lh
    // of fragment i's row (no zero points: zp = 8).
    auto read_sz = [&](int buf, h2_t (&S2)[FN][2], h2_t (&ZB)[FN][2]) {
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const int rr = wn * 128 + 32 * i + lr;
            const floatx4_t sc = *reinterpret_cast<const floatx4_t*>(lds + OFF_S + buf * SG + rr * 16);
            // The 2-byte load leaves the slot's upper half as it was: keep the low 16 bits.
            const uint32_t z = *reinterpret_cast<const uint32_t*>(lds + OFF_Z + buf * ZG + rr * 4) & 0xFFFFu;
            const uint32_t zl = (p.zp ? z : 0x8888u) >> (4 * lh);
            const uint32_t zd = zl | (zl << 16);
            const _Float16 s0 = (_Float16)(lh ? sc[1] : sc[0]), s1 = (_Float16)(lh ? sc[3] : sc[2]);
            S2[i][0] = h2_t{s0, s0};
            S2[i][1] = h2_t{s1, s1};
            ZB[i][0] = as_h2(and_or(zd, 0x000F000Fu, kHalfMagic));
            ZB[i][1] = as_h2(and_or(zd >> 8, 0x000F000Fu, kHalfMagic));
        }
    };
    // B operands (both sub-steps) of one fragment for step ph of its group.
    auto dequant_frag = [&](const u32x4_t& rc, h2_t s2, h2_t zb, auto phc, half8_t (&b)[2]) {
        constexpr int ph = decltype(phc)::value;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            uint32_t o[4];
            dequant8_f16(rc[2 * (ph & 1) + sub], zb, s2, o);
            b[sub] = __builtin_bit_cast(half8_t, u32x4_t{o[0], o[1], o[2], o[3]});
        }
    };

    floatx16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = floatx16_t{};
    }
    // A operands of one sub-step (16 k) of step stage st.
    auto load_a = [&](int st, int sub, half8_t (&a)[FM]) {
        const uint8_t* As = lds + OFF_A + st * A_ST;
        const int j = 2 * lh + sub;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int r = wm * 128 + 32 * i + lr;
            a[i] = *reinterpret_cast<const half8_t*>(As + r * 64 + pipe_slot(r, j) * 16);
        }
    };
    auto mfma_ops = [&](const half8_t (&a)[FM], const half8_t (&b)[FN][2], int sub) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int jn = 0; jn < FN; ++jn)
                acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[jn][sub], acc[i][jn], 0, 0, 0);
        }
    };

    // Registers carried between steps:
    //   a0      A operands of the first sub-step of the current step (read in the previous
    //           step's second half);
    //   bq[x]   B operands of the steps with parity x: step t uses bq[t & 1] and, during
    //           its MFMAs, dequantizes step t+1 into bq[(t + 1) & 1];
    //   rcA/rcB code chunks of the pairs of steps (0,1) / (2,3) of a group: rcB (group g)
    //           is read at step 4g, rcA of group g+1 at step 4g+2, each a step before the
    //           dequant that first needs it;
    //   S2/ZB   packed scales and zero points of the current group, S2n/ZBn of the next
    //           (read at step 4g+2, used from the dequant of step 4g+4 on).
    // Step t (ph = t % 4), R1 = A operands of its second sub-step:
    //   first half:  read R1 (and rcB at ph 0, rcA at ph 2); MFMAs on a0, interleaved with
    //                the dequant of fragments 0-1 of step t+1; wait for A(t+1); barrier;
    //   second half: read a0 of step t+1 (and scn/zwn at ph 2); MFMAs on R1, interleaved
    //                with the dequant of fragments 2-3 and the issue of A(t+3) and, at
    //                ph 0, of weight group t/4 + 2.
    // Raw-buffer lifetime: group g-1's buffer is last read in the first half of step 4g-4
    // (its rcB; its rcA and scales at 4g-6), and group g+2 overwrites it after the barrier
    // of step 4g.
    half8_t a0[FM];
    half8_t bq[2][FN][2];
    u32x4_t rcA[FN], rcB[FN];
    h2_t S2[FN][2], ZB[FN][2], S2n[FN][2], ZBn[FN][2];

    issue_b(0, 0);
    issue_b(1, 1);
    issue_a(0, 0);
    issue_a(1, 1);
    issue_a(2, 2);
    wait_vmcnt<8>();                     // B(0), B(1), A(0): then A(1), A(2)
    lds_barrier();                       // every wave's rows of B(0) and A(0)
    read_codes(0, 0, rcA);
    read_sz(0, S2, ZB);
#pragma unroll
    for (int i = 0; i < FN; ++i) dequant_frag(rcA[i], S2[i][0], ZB[i][0], std::integral_constant<int, 0>{}, bq[0][i]);
    load_a(0, 0, a0);

    auto step = [&](int t, auto phase, auto wait, int bcur, int bnext, int nbuf) {
        constexpr int ph = decltype(phase)::value, ph1 = (ph + 1) & 3;
        constexpr int par = ph & 1, npar = ph1 & 1;
        using PH1 = std::integral_constant<int, ph1>;
        __builtin_amdgcn_sched_barrier(0);
        half8_t a1[FM];
        load_a(ph, 1, a1);
        if constexpr (ph == 0) read_codes(bcur, 1, rcB);
        if constexpr (ph == 2) read_codes(bnext, 0, rcA);
        // The dequant of step t+1: codes of its pair, scales of its group.
        auto& rcn = [&]() -> u32x4_t(&)[FN] { if constexpr (ph1 < 2) return rcA; else return rcB; }();
        auto& S2x = [&]() -> h2_t(&)[FN][2] { if constexpr (ph == 3) return S2n; else return S2; }();
        auto& ZBx = [&]() -> h2_t(&)[FN][2] { if constexpr (ph == 3) return ZBn; else return ZB; }();
        mfma_ops(a0, bq[par], 0);
#pragma unroll
        for (int i = 0; i < 2; ++i) dequant_frag(rcn[i], S2x[i][ph1 >> 1], ZBx[i][ph1 >> 1], PH1{}, bq[npar][i]);
        constexpr int nr0 = (ph == 0 || ph == 2) ? 8 : 4;
#pragma unroll
        for (int g = 0; g < nr0; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        }
#pragma unroll
        for (int g = nr0; g < 16; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<decltype(wait)::value>();
        lds_barrier();
        load_a((ph + 1) & 3, 0, a0);
        if constexpr (ph == 2) read_sz(bnext, S2n, ZBn);
        mfma_ops(a1, bq[par], 1);
#pragma unroll
        for (int i = 2; i < FN; ++i) dequant_frag(rcn[i], S2x[i][ph1 >> 1], ZBx[i][ph1 >> 1], PH1{}, bq[npar][i]);
        issue_a(t + 3, (ph + 3) & 3);
        if constexpr (ph == 0) issue_b((t >> 2) + 2, nbuf);
        constexpr int nr1 = ph == 2 ? 12 : 4;
#pragma unroll
        for (int g = 0; g < nr1; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        }
#pragma unroll
        for (int g = nr1; g < 16; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (ph == 3) {
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                S2[i][0] = S2n[i][0];
                S2[i][1] = S2n[i][1];
                ZB[i][0] = ZBn[i][0];
                ZB[i][1] = ZBn[i][1];
            }
        }
    };
    using std::integral_constant;
    int b0 = 0, b1 = 1, b2 = 2;           // raw buffers of groups g, g+1, g+2
    for (int t = 0; t < nsteps; t += 4) {
        step(t, integral_constant<int, 0>{}, integral_constant<int, 4>{}, b0, b1, b2);       // A(t+1): then A(t+2)
        step(t + 1, integral_constant<int, 1>{}, integral_constant<int, 10>{}, b0, b1, b2);  // A(t+2): then A(t+3), B(g+2)
        step(t + 2, integral_constant<int, 2>{}, integral_constant<int, 10>{}, b0, b1, b2);  // A(t+3): then B(g+2), A(t+4)
        step(t + 3, integral_constant<int, 3>{}, integral_constant<int, 4>{}, b0, b1, b2);   // A(t+4): then A(t+5)
        const int bt = b0;
        b0 = b1;
        b1 = b2;
        b2 = bt;
    }
    wait_vmcnt<0>();
    pipe_epilogue(p, it, acc);
}

}  // namespace msnb
