// Device-side helpers shared by the verify-step kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.hpp"

namespace kyro {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ void latch_error(int* err, int bits) { atomicOr(err, bits); }

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two floats -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 h;
    h[0] = (__bf16)lo;
    h[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, h);
}

// 2^x with v_exp_f32 directly (outputs below 2^-126 flush to zero, which softmax tolerates).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Cross-lane moves. xor 16 / xor 32 swap the 16-lane rows of a wave64.
__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, 64); }

// Max over the four 16-lane rows of a wave64 (lanes l, l ^ 16, l ^ 32 and l ^ 48), in every lane.
// permlane16_swap(v, v) returns {v of lane l with rows 1 and 3 replaced by rows 0 and 2, v with
// rows 0 and 2 replaced by rows 1 and 3}, so the max of the pair is the max over rows 2i, 2i + 1;
// permlane32_swap does the same for the halves. Two VALU swaps where __shfl_xor makes two round
// trips through the LDS unit.
__device__ __forceinline__ float max_over_rows(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Sum over each 16-lane row with DPP; every lane of the row gets the row total.
__device__ __forceinline__ float row16_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));  // row_mirror
    return v;
}

// Sum over each 8-lane half-row with DPP; every lane of the half-row gets its total.
__device__ __forceinline__ float row8_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
    return v;
}

// DPP copy of v from another lane (ctrl: a DPP control code, rmask: the 16-lane rows written);
// lanes whose source lies outside the row, or rows outside rmask, get 0.
#define KYRO_DPP(v, ctrl, rmask) __builtin_amdgcn_update_dpp(0, (v), (ctrl), (rmask), 0xf, false)

// Inclusive wave scans with DPP: row_shr 1, 2, 4, 8 inside each 16-lane row, then row_bcast:15
// (rows 1 and 3 add lane 15 of the row before) and row_bcast:31 (rows 2 and 3 add lane 31).
// STEP(ctrl, rmask) adds one shifted copy.
#define KYRO_DPP_SCAN(STEP) \
    STEP(0x111, 0xf);       \
    STEP(0x112, 0xf);       \
    STEP(0x114, 0xf);       \
    STEP(0x118, 0xf);       \
    STEP(0x142, 0xa);       \
    STEP(0x143, 0xc)

__device__ __forceinline__ float wave_incl_scan_f(float x) {
#define KYRO_STEP_F(ctrl, rmask) x += __int_as_float(KYRO_DPP(__float_as_int(x), ctrl, rmask))
    KYRO_DPP_SCAN(KYRO_STEP_F);
#undef KYRO_STEP_F
    return x;
}

__device__ __forceinline__ int wave_incl_scan_i(int x) {
#define KYRO_STEP_I(ctrl, rmask) x += KYRO_DPP(x, ctrl, rmask)
    KYRO_DPP_SCAN(KYRO_STEP_I);
#undef KYRO_STEP_I
    return x;
}

// Lane l's float as a scalar (the builtin is typed int: the bits move, not a converted value).
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Wave reductions: the 16-lane rows with DPP, then the four row results read as scalars (every
// lane gets the same value).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __int_as_float(KYRO_DPP(__float_as_int(v), 0xB1, 0xF)));   // quad_perm [1,0,3,2]
    v = fmaxf(v, __int_as_float(KYRO_DPP(__float_as_int(v), 0x4E, 0xF)));   // quad_perm [2,3,0,1]
    v = fmaxf(v, __int_as_float(KYRO_DPP(__float_as_int(v), 0x141, 0xF)));  // row_half_mirror
    v = fmaxf(v, __int_as_float(KYRO_DPP(__float_as_int(v), 0x140, 0xF)));  // row_mirror
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

__device__ __forceinline__ uint4 load16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

}  // namespace kyro
