// nbits_device.h — device-side helpers shared by the MatMulNBits kernels.
//
// Dequantization is W[n,k] = ((float)q - zp) * scale with q the 4-bit code of
// column k in row n and zp an integer, as in
// src/ModelSharp/Cpu/Kernels/Quantize/MatMulNBitsSimd.cs:100-111. For integer
// zp, q - zp is exact, so the product is the only rounding. The library is
// compiled with -ffp-contract=off, so that product is never fused into the
// accumulation that follows it; the accumulations are explicit fmaf.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace msnb {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;             // CDNA wavefront
constexpr uint32_t kHalfMagic = 0x64006400u;   // two fp16 1024.0: 1024 + v for a 10-bit v

__device__ __forceinline__ h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }

__device__ __forceinline__ uint32_t as_u32(h2_t v) { return __builtin_bit_cast(uint32_t, v); }

// (x & mask) | orv in one VALU op. gfx9 VOP3 takes no literal and at most one
// scalar operand, so the mask rides in an SGPR and orv in a VGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t orv)
{
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(orv));
    return r;
}

// fp32 fma(fp16 lane of h2 widened, s, c): with c = -0.0 (the additive
// identity) this is the single rounding of (float)h * s.
__device__ __forceinline__ float mix_lo(uint32_t h2, float s, float c)
{
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(s), "s"(c));
    return r;
}
__device__ __forceinline__ float mix_hi(uint32_t h2, float s, float c)
{
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(s), "s"(c));
    return r;
}

// Per-block dequant constants. A 4-bit code sitting in bits 0-3 of an fp16
// lane with exponent bits 0x6400 reads as 1024 + q; sitting in bits 4-7 it
// reads as 1024 + 16q. Subtracting 1024 + zp (resp. 1024 + 16zp) in packed fp16
// is exact and leaves d = q - zp (resp. 16(q - zp)); the fp32 product with s
// (resp. s/16, exact by a power of two for |s| >= 2^-122) is then the single
// rounding of (q - zp) * s.
struct BlockDq {
    h2_t zb;     // (1024 + zp) x2
    h2_t zb16;   // (1024 + 16 zp) x2
    float s;     // scale
    float s16;   // scale / 16
};

__device__ __forceinline__ BlockDq block_dq(int zp, float s)
{
    BlockDq q;
    q.zb = as_h2(kHalfMagic | ((uint32_t)zp << 16) | (uint32_t)zp);
    q.zb16 = as_h2(kHalfMagic | ((uint32_t)zp << 20) | ((uint32_t)zp << 4));
    q.s = s;
    q.s16 = s * 0.0625f;
    return q;
}

// Dequantizes the eight 4-bit codes of one little-endian dword (codes for
// k = 8j .. 8j+7 of a chunk: byte i holds k=2i in its low nibble and k=2i+1 in
// its high nibble) to fp32, w[i] for k = 8j + i. 25 VALU ops for 8 weights:
// one shift, four and_or, four packed fp16 subtracts, eight fma_mix.
__device__ __forceinline__ void dequant8(uint32_t x, const BlockDq& q, float (&w)[8])
{
    const uint32_t magic = kHalfMagic;
    const uint32_t x8 = x >> 8;
    const uint32_t d0 = as_u32(as_h2(and_or(x, 0x000F000Fu, magic)) - q.zb);      // k0, k4
    const uint32_t d1 = as_u32(as_h2(and_or(x, 0x00F000F0u, magic)) - q.zb16);    // 16*k1, 16*k5
    const uint32_t d2 = as_u32(as_h2(and_or(x8, 0x000F000Fu, magic)) - q.zb);     // k2, k6
    const uint32_t d3 = as_u32(as_h2(and_or(x8, 0x00F000F0u, magic)) - q.zb16);   // 16*k3, 16*k7
    const float nz = -0.0f;
    w[0] = mix_lo(d0, q.s, nz);
    w[4] = mix_hi(d0, q.s, nz);
    w[1] = mix_lo(d1, q.s16, nz);
    w[5] = mix_hi(d1, q.s16, nz);
    w[2] = mix_lo(d2, q.s, nz);
    w[6] = mix_hi(d2, q.s, nz);
    w[3] = mix_lo(d3, q.s16, nz);
    w[7] = mix_hi(d3, q.s16, nz);
}

// acc + (float)h * a for the low / high fp16 lane of h2: an fp32 fma of the
// widened half (exact) — selected as one v_fma_mix_f32. Written in C++, not
// asm, so the scheduler can hoist the activation loads feeding it.
__device__ __forceinline__ float fmac_lo(uint32_t h2, float a, float acc)
{
    return __builtin_fmaf((float)as_h2(h2).x, a, acc);
}
__device__ __forceinline__ float fmac_hi(uint32_t h2, float a, float acc)
{
    return __builtin_fmaf((float)as_h2(h2).y, a, acc);
}

// The exact differences of one dword of codes as four fp16 pairs:
// d[0] = (k0, k4), d[1] = 16*(k1, k5), d[2] = (k2, k6), d[3] = 16*(k3, k7),
// each k standing for q_k - zp. 9 VALU ops.
__device__ __forceinline__ void diffs8(uint32_t x, h2_t zb, h2_t zb16, uint32_t (&d)[4])
{
    const uint32_t magic = kHalfMagic;
    const uint32_t x8 = x >> 8;
    d[0] = as_u32(as_h2(and_or(x, 0x000F000Fu, magic)) - zb);
    d[1] = as_u32(as_h2(and_or(x, 0x00F000F0u, magic)) - zb16);
    d[2] = as_u32(as_h2(and_or(x8, 0x000F000Fu, magic)) - zb);
    d[3] = as_u32(as_h2(and_or(x8, 0x00F000F0u, magic)) - zb16);
}

// acc + sum_i (q_i - zp) * a_i over the 8 codes whose diffs8() are d, with the
// activations a0 = a[k0..k3], a1 = a[k4..k7] staged with the odd k pre-divided
// by 16 (exact: a power of two), which cancels the 16 in d[1], d[3]. Every
// product is exact inside the fma; one rounding per accumulation.
__device__ __forceinline__ float dot8(const uint32_t (&d)[4], const float4& a0, const float4& a1, float acc)
{
    acc = fmac_lo(d[0], a0.x, acc);
    acc = fmac_lo(d[1], a0.y, acc);
    acc = fmac_lo(d[2], a0.z, acc);
    acc = fmac_lo(d[3], a0.w, acc);
    acc = fmac_hi(d[0], a1.x, acc);
    acc = fmac_hi(d[1], a1.y, acc);
    acc = fmac_hi(d[2], a1.z, acc);
    acc = fmac_hi(d[3], a1.w, acc);
    return acc;
}

// ---- shared by the GEMV kernels ---------------------------------------------------
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
// A staged activation chunk in LDS: 32 activations pre-scaled (even k by 2^24, odd
// k by 2^20) in 8 float4, then (sum of the 32 unscaled activations, 0, 0, 0). The
// ninth float4 also pads the chunk stride off a power of two (fewer bank conflicts).
constexpr int kChunkStride4 = 9;
// A buffer offset beyond every resource the kernels build: a load from it returns
// zero and makes no memory request.
constexpr int kOOB = 0x7ffffff0;
constexpr uint32_t kBufferWord3 = 0x00020000u;   // raw buffer resource, gfx9 data format
constexpr float kTwo24 = 16777216.0f;            // 2^24
constexpr float kTwo20 = 1048576.0f;             // 2^20


__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, (int)kBufferWord3);
}

// Buffer cache policy sc1 (device scope): stores write through to where every XCD
// reads, loads do not return another XCD's stale copy.
constexpr int kDeviceCoherent = 16;
// Buffer cache policy nt: streaming data, not kept in the caches for reuse.
constexpr int kNonTemporal = 2;

// x + (x moved by one DPP control); lanes whose source is outside the row, or whose row the
// mask leaves out, add 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float x)
{
    const int y = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xF, false);
    return x + __builtin_bit_cast(float, y);
}

// Maximum of x over each aligned 16-lane row, in every lane of the row: quad_perm swaps
// of neighbours and pairs (every lane then holds its quad's maximum), row_half_mirror
// (lane i of each 8-lane half with lane 7 - i: the other quad), row_mirror (lane i with
// lane 15 - i: the other half). Four VALU ops instead of four ds_bpermute round trips.
template <int CTRL>
__device__ __forceinline__ float dpp_read(float x)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max_all(float x)
{
    x = fmaxf(x, dpp_read<0xB1>(x));    // quad_perm [1,0,3,2]
    x = fmaxf(x, dpp_read<0x4E>(x));    // quad_perm [2,3,0,1]
    x = fmaxf(x, dpp_read<0x141>(x));   // row_half_mirror
    x = fmaxf(x, dpp_read<0x140>(x));   // row_mirror
    return x;
}

// Sum of x over each aligned group of G lanes (G = 16, 32 or 64), left in the group's last
// lane (the other lanes hold partial sums): an inclusive scan inside each 16-lane row
// (row_shr 1, 2, 4, 8), then row_bcast:15 into rows 1 and 3 and row_bcast:31 into rows 2
// and 3. Every step is one VALU op; a ds_bpermute butterfly costs an LDS round trip per
// level. The order of the additions is fixed, so results are deterministic.
template <int G>
__device__ __forceinline__ float group_sum_to_last(float x)
{
    static_assert(G == 16 || G == 32 || G == 64, "groups of 16, 32 or 64 lanes");
    x = dpp_add<0x111, 0xF>(x);   // row_shr:1
    x = dpp_add<0x112, 0xF>(x);   // row_shr:2
    x = dpp_add<0x114, 0xF>(x);   // row_shr:4
    x = dpp_add<0x118, 0xF>(x);   // row_shr:8
    if constexpr (G >= 32) x = dpp_add<0x142, 0xA>(x);   // row_bcast:15 -> rows 1, 3
    if constexpr (G == 64) x = dpp_add<0x143, 0xC>(x);   // row_bcast:31 -> rows 2, 3
    return x;
}

// Cross-workgroup hand-off through data written and read with agent-scope atomic
// stores / loads (those write and read through the caches, so the data needs no L2
// write-back or invalidate). These two only order: the release form waits until every
// earlier vector memory operation of the wave has completed, the acquire form keeps
// later loads behind the atomic it follows. (An agent-scope fence would also write back
// or invalidate the XCD's whole L2, which costs microseconds per workgroup.)
__device__ __forceinline__ void wait_vmem_order_only_release()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xF << 8));   // vmcnt(0) expcnt(7) lgkmcnt(15)
}
__device__ __forceinline__ void wait_vmem_order_only_acquire()
{
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xF << 8));
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// acc + a * (fp16 lane widened) — one v_fma_mix_f32.
__device__ __forceinline__ float mix_lo_acc(uint32_t h2, float a, float acc)
{
    return __builtin_fmaf((float)as_h2(h2).x, a, acc);
}
__device__ __forceinline__ float mix_hi_acc(uint32_t h2, float a, float acc)
{
    return __builtin_fmaf((float)as_h2(h2).y, a, acc);
}

// The four masked code pairs of dword x: p[0] = (k0, k4) and p[2] = (k2, k6) as
// q * 2^-24, p[1] = (k1, k5) and p[3] = (k3, k7) as 16 q * 2^-24.
__device__ __forceinline__ void code_pairs(uint32_t x, uint32_t (&p)[4])
{
    const uint32_t x8 = x >> 8;
    p[0] = x & 0x000F000Fu;
    p[1] = x & 0x00F000F0u;
    p[2] = x8 & 0x000F000Fu;
    p[3] = x8 & 0x00F000F0u;
}

// Packed zero point of block `blk` from a row of packed nibbles
// (MatMulNBitsKernel.cs:349-356 with bits=4).
__device__ __forceinline__ int zp_nibble(const uint8_t* zrow, int blk)
{
    return (zrow[blk >> 1] >> ((blk & 1) * 4)) & 0x0F;
}

// acc + sum of a_k q_k over the 8 codes of one dword whose code_pairs() are p,
// with a0 = a'[k0..k3], a1 = a'[k4..k7] staged pre-scaled. Every product is exact
// inside its fma; one rounding per accumulation.
__device__ __forceinline__ float qdot8(const uint32_t (&p)[4], const float4& a0, const float4& a1, float acc)
{
    acc = mix_lo_acc(p[0], a0.x, acc);
    acc = mix_lo_acc(p[1], a0.y, acc);
    acc = mix_lo_acc(p[2], a0.z, acc);
    acc = mix_lo_acc(p[3], a0.w, acc);
    acc = mix_hi_acc(p[0], a1.x, acc);
    acc = mix_hi_acc(p[1], a1.y, acc);
    acc = mix_hi_acc(p[2], a1.z, acc);
    acc = mix_hi_acc(p[3], a1.w, acc);
    return acc;
}

}  // namespace msnb
