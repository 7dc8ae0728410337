// nbits_device.h — device-side helpers shared by the MatMulNBits kernels.
//
// Dequantization is W[n,k] = ((float)q - zp) * scale with q the 4-bit code of
// column k in row n and zp an integer, as in
// src/ModelSharp/Cpu/Kernels/Quantize/MatMulNBitsSimd.cs:100-111. For integer
// zp, q - zp is exact (the kernels form it in fp16 with the packed-half trick
// below), so the product with the scale is the only rounding. The library is
// compiled with -ffp-contract=off, so no product is fused into the accumulation
// that follows it; the accumulations are explicit fmaf.
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

// (1024 + zp, 1024 + zp) and (1024 + 16 zp, 1024 + 16 zp) as fp16 pairs, the subtrahends
// of diffs8() for a 4-bit zero point.
__device__ __forceinline__ h2_t zp_half2(uint32_t zp) { return as_h2(kHalfMagic | (zp << 16) | zp); }
__device__ __forceinline__ h2_t zp16_half2(uint32_t zp) { return as_h2(kHalfMagic | (zp << 20) | (zp << 4)); }

// Activations staged for dot8(): the odd k (y, w of a float4 of k = 4i .. 4i+3) divided
// by 16, exactly (a power of two).
__device__ __forceinline__ float4 stage_odd16(const float4& v)
{
    return float4{v.x, v.y * 0.0625f, v.z, v.w * 0.0625f};
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
// A staged activation chunk in LDS: 32 activations (odd k divided by 16) in 8 float4,
// then one float4 of padding that keeps the chunk stride off a power of two (fewer bank
// conflicts).
constexpr int kChunkStride4 = 9;
// A buffer offset beyond every resource the kernels build: a load from it returns
// zero and makes no memory request.
constexpr int kOOB = 0x7ffffff0;
constexpr uint32_t kBufferWord3 = 0x00020000u;   // raw buffer resource, gfx9 data format


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
// x of lane l (a wave-uniform index), in every lane: v_readlane into a scalar register.
__device__ __forceinline__ float lane_value(float x, int l)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}
__device__ __forceinline__ float row16_max_all(float x)
{
    x = fmaxf(x, dpp_read<0xB1>(x));    // quad_perm [1,0,3,2]
    x = fmaxf(x, dpp_read<0x4E>(x));    // quad_perm [2,3,0,1]
    x = fmaxf(x, dpp_read<0x141>(x));   // row_half_mirror
    x = fmaxf(x, dpp_read<0x140>(x));   // row_mirror
    return x;
}

// x of lane l ^ 16 (the same position in the other 16-lane row of the half) by
// v_permlane16_swap: with x on both sides, the first result holds rows 0 and 2 in rows 1
// and 3, the second rows 1 and 3 in rows 0 and 2. A VALU op, where ds_bpermute is an LDS
// round trip.
__device__ __forceinline__ float xor16_value(float x)
{
    const int xi = __builtin_bit_cast(int, x);
    const auto sw = __builtin_amdgcn_permlane16_swap(xi, xi, false, false);
    return __builtin_bit_cast(float, (threadIdx.x & 16) ? sw[0] : sw[1]);
}
// x of lane l ^ 32 (the other half of the wave) by v_permlane32_swap: the first result
// holds the lower half in the upper, the second the upper half in the lower.
__device__ __forceinline__ float xor32_value(float x)
{
    const int xi = __builtin_bit_cast(int, x);
    const auto sw = __builtin_amdgcn_permlane32_swap(xi, xi, false, false);
    return __builtin_bit_cast(float, (threadIdx.x & 32) ? sw[0] : sw[1]);
}
// Maximum of x over each aligned 32-lane half of the wave, in every lane of the half.
__device__ __forceinline__ float half_max_all(float x)
{
    x = row16_max_all(x);
    return fmaxf(x, xor16_value(x));
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

// Sum of x over each aligned 32-lane half of the wave, in every lane of the half (fixed
// order: the scan of group_sum_to_last, then the halves' last lanes read back).
__device__ __forceinline__ float half_sum_all(float x)
{
    x = group_sum_to_last<32>(x);
    const float lo = lane_value(x, 31), hi = lane_value(x, 63);
    return (threadIdx.x & 32) ? hi : lo;
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

// Packed zero point of block `blk` from a row of packed nibbles
// (MatMulNBitsKernel.cs:349-356 with bits=4).
__device__ __forceinline__ int zp_nibble(const uint8_t* zrow, int blk)
{
    return (zrow[blk >> 1] >> ((blk & 1) * 4)) & 0x0F;
}

}  // namespace msnb
