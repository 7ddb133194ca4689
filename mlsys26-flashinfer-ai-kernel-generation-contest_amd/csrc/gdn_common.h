// Shared device helpers for the gfx950 Gated DeltaNet kernels: bf16 conversion,
// wavefront reductions on DPP, vector types, and the host-side error channel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdn_hip.h"

namespace gdn {

typedef uint16_t bf16_t;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint32_t h)
{
    return __uint_as_float(h << 16);
}

// Low / high bf16 of a packed pair -> float (exact).
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 pair (lo = a, hi = b), round to nearest even: one
// v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2_t));
}

// float -> bf16 bits (round to nearest even), in the low 16 bits.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) { return pack_bf16x2(f, 0.f) & 0xffffu; }

// Split two floats into bf16 hi = bf16(x) and lo = bf16(x - hi), both packed as pairs.
__device__ __forceinline__ void split_bf16x2(float a, float b, uint32_t &hi, uint32_t &lo)
{
    hi = pack_bf16x2(a, b);
    lo = pack_bf16x2(a - bf16lo(hi), b - bf16hi(hi));
}

// The same split with each residual x - bf16(x) formed by one dot product,
// v_dot2c_f32_bf16: hi . {-1, 0} + a and hi . {0, -1} + b (exact: the residual is an fp32
// value). The instruction accumulates into its destination, so the split writes a and b's
// registers when they die there. The two multipliers are kept in SGPRs, made once per kernel
// by split_consts(): left as immediates, the compiler encodes {-1, 0} as the inline
// constant -1.0, which the hardware reads as the fp32 pattern 0xbf800000, i.e. {0, -1}
// (checked on MI355X over 2^20 inputs: every residual of the SGPR form matches a - bf16(a)
// bit for bit; the immediate form gets almost all of them wrong).
struct SplitConsts {
    bf16x2_t m0, m1;
};
__device__ __forceinline__ SplitConsts split_consts()
{
    uint32_t m0 = 0x0000bf80u, m1 = 0xbf800000u;  // {-1, 0}, {0, -1}
    asm volatile("" : "+s"(m0), "+s"(m1));
    return SplitConsts{__builtin_bit_cast(bf16x2_t, m0), __builtin_bit_cast(bf16x2_t, m1)};
}
__device__ __forceinline__ void split_bf16x2(float a, float b, uint32_t &hi, uint32_t &lo,
                                             const SplitConsts &k)
{
    hi = pack_bf16x2(a, b);
    const bf16x2_t h = __builtin_bit_cast(bf16x2_t, hi);
    lo = pack_bf16x2(__builtin_amdgcn_fdot2_f32_bf16(h, k.m0, a, false),
                     __builtin_amdgcn_fdot2_f32_bf16(h, k.m1, b, false));
}

// DPP control words (GCN/CDNA encoding).
constexpr int kDppQuadXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;  // lane i <- lane 7-i within each 8 lanes
constexpr int kDppRowMirror = 0x140;      // lane i <- lane 15-i within each 16 lanes

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over each aligned group of 8 lanes; every lane of the group receives the
// same bits (the adds pair operands symmetrically).
__device__ __forceinline__ float group8_sum(float x)
{
    x += dpp_mov<kDppRowHalfMirror>(x);
    x += dpp_mov<kDppQuadXor1>(x);
    x += dpp_mov<kDppQuadXor2>(x);
    return x;
}

// Sum over each aligned group of 16 lanes.
__device__ __forceinline__ float group16_sum(float x)
{
    x += dpp_mov<kDppRowMirror>(x);
    return group8_sum(x);
}

}  // namespace gdn

// Host-side error channel (gdn_abi.hip).
int gdn_set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int gdn_check_launch(const char *what);
// Start of every C-ABI entry point: clears the last-error message.
void gdn_begin_call();
// After argument checks, before the first launch: drains a stale HIP error.
void gdn_begin_launches();
