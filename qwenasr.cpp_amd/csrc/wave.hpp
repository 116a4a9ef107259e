// Wavefront reductions on DPP (gfx950, wave64), for device code only.
//
// Four in-row steps -- quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror -- leave
// every lane of each 16-lane row with the row's total (each step adds two partial sums in both lanes,
// and a + b == b + a, so all 16 lanes hold the same bits).  row_bcast:15 then combines row 0 into row 1
// and row 2 into row 3, and row_bcast:31 combines rows 0 + 1 into row 3, so lane 63 ends with
// (r3 + r2) + (r1 + r0).  The *_all variants broadcast lane 63 with readlane.  Every step is a VALU
// operation: no LDS round trip (a __shfl_xor butterfly costs one ds_bpermute wait per step).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace qa {

template <int CTRL>
__device__ inline float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

// DPP source in the rows selected by ROWS, `other` in the remaining rows.
template <int CTRL, int ROWS>
__device__ inline float dpp_rows_f(float v, float other) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(other), __float_as_int(v), CTRL, ROWS, 0xf, false));
}

template <int CTRL>
__device__ inline double dpp_d(double v) {
    const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
    const uint32_t lo = __builtin_amdgcn_mov_dpp(static_cast<int>(static_cast<uint32_t>(u)), CTRL, 0xf, 0xf, false);
    const uint32_t hi = __builtin_amdgcn_mov_dpp(static_cast<int>(static_cast<uint32_t>(u >> 32)), CTRL, 0xf, 0xf, false);
    return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

template <int CTRL, int ROWS>
__device__ inline double dpp_rows_zero_d(double v) {   // 0.0 in the rows outside ROWS
    const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
    const uint32_t lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u)), CTRL, ROWS, 0xf, false);
    const uint32_t hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u >> 32)), CTRL, ROWS, 0xf, false);
    return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

__device__ inline float bcast63_f(float v) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63)); }

__device__ inline double bcast63_d(double v) {
    const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(u)), 63);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(u >> 32)), 63);
    return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

// Sum over the 16 lanes of each row, in every lane of the row.
__device__ inline float row_sum16_f(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    return v;
}

__device__ inline float wave_sum_lane63(float v) {
    v = row_sum16_f(v);
    v += dpp_rows_f<0x142, 0xa>(v, 0.0f);
    v += dpp_rows_f<0x143, 0xc>(v, 0.0f);
    return v;
}

__device__ inline float wave_max_lane63(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    v = fmaxf(v, dpp_rows_f<0x142, 0xa>(v, -INFINITY));
    v = fmaxf(v, dpp_rows_f<0x143, 0xc>(v, -INFINITY));
    return v;
}

__device__ inline double wave_sum_d_lane63(double v) {
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    v += dpp_d<0x141>(v);
    v += dpp_d<0x140>(v);
    v += dpp_rows_zero_d<0x142, 0xa>(v);
    v += dpp_rows_zero_d<0x143, 0xc>(v);
    return v;
}

__device__ inline float wave_sum_all(float v) { return bcast63_f(wave_sum_lane63(v)); }
__device__ inline float wave_max_all(float v) { return bcast63_f(wave_max_lane63(v)); }
__device__ inline double wave_sum_d_all(double v) { return bcast63_d(wave_sum_d_lane63(v)); }

}  // namespace qa
