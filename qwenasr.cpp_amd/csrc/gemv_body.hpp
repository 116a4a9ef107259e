// Batch-1 GEMV of the decode step as a device function, shared by the one-GEMV-per-launch kernel
// (decoder_ops.hip) and the persistent decode step (decode_persist.hip), so that both compute every
// output with the same instructions in the same order.
//
// y[o] (+)= sum_k W[o][k] * x'[k] with x' = x or RMSNorm(x) * norm_w (PRENORM), epilogues: store,
// residual accumulate, silu(gate) * up.  Replaces linear_ggml with PREC_F32 and the rms_norm / mul /
// silu / add nodes around it (text-decoder.cpp:83-90, 365-373, 465-493).
#pragma once

#include "coherent.hpp"
#include "common.hpp"
#include "wave.hpp"

namespace qa {
namespace {

enum { kEpiStore = 0, kEpiAccum = 1, kEpiSwiglu = 2 };

struct GemvParams {
    const void * W;         // [rows_w][in_dim] f32, or bf16 bits (B16); for SwiGLU rows_w = 2 * out_dim
                            // (gate rows, then up rows)
    const float * x;        // [in_dim]
    float * y;              // [out_dim]
    const float * norm_w;   // pre-RMSNorm weight (PRENORM only)
    int32_t out_dim, in_dim;
    float eps;
    const float * res;      // kEpiAccum: the residual rows added to (y itself in the per-launch kernel)
};


typedef float f4 __attribute__((ext_vector_type(4)));

__device__ inline float dot4(const f4 a, const f4 b, float acc) {
    acc = fmaf(a.x, b.x, acc);
    acc = fmaf(a.y, b.y, acc);
    acc = fmaf(a.z, b.z, acc);
    acc = fmaf(a.w, b.w, acc);
    return acc;
}

typedef unsigned int u2 __attribute__((ext_vector_type(2)));

// four bf16 values (little-endian: element 0 in the low half of .x) widened to the f32 values whose
// high halves they are
__device__ inline f4 widen_bf16x4(const u2 b) {
    f4 r;
    r.x = __uint_as_float(b.x << 16);
    r.y = __uint_as_float(b.x & 0xffff0000u);
    r.z = __uint_as_float(b.y << 16);
    r.w = __uint_as_float(b.y & 0xffff0000u);
    return r;
}

// IN4 = in_dim / 256 (each lane holds 4 * IN4 input elements), NR rows per wave iteration.  `block` and
// `n_blocks` take the place of blockIdx.x and gridDim.x: waves walk the rows grid-stride.
// Load order: x and the norm weight first, then the weight rows of the wave's first iteration, so the
// RMSNorm of x (which waits for its own loads only: vector loads complete in issue order) runs while
// the weight rows stream in.  Rows past out_dim re-read the last row and are not stored.
// B16: W holds bf16 bits; lane l reads elements k 256 + 4 l .. + 3 as one 8-byte load where the f32
// kernel reads them as one 16-byte load, so both kernels assign every element to the same lane, step
// and fmaf.
// COH: y is written with agent-scope (write-through) stores, for workgroups of the same launch on other
// XCDs (coherent.hpp); inputs are plain loads.
template <int IN4, int NR, int EPI, bool PRENORM, bool B16, bool COH>
__device__ __forceinline__ void gemv_body(const GemvParams & p, int block, int n_blocks) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int gw = block * 4 + wave;
    const int nw = n_blocks * 4;
    const int64_t in = p.in_dim;
    // x is staged once per workgroup and shared through LDS: wave w loads (and, PRENORM, normalises)
    // the steps k = w QK .. w QK + QK - 1 of x and of the norm weight, a quarter each, instead of every
    // wave loading all of both (x alone is as many bytes per wave as its two bf16 weight rows).
    // Measured on the config-3 decode step: 1.136 -> 1.084 ms per token for the RMSNorm GEMVs, then
    // 1.086 -> 1.068 for the others.
    constexpr int QK = IN4 / 4;
    static_assert(IN4 % 4 == 0, "staging x needs in_dim a multiple of 1024");
    const int k0 = wave * QK;
    f4 xv[IN4], nv[QK];
#pragma unroll
    for (int k = 0; k < QK; ++k) xv[k] = *reinterpret_cast<const f4 *>(p.x + (k0 + k) * 256 + lane * 4);
    if (PRENORM) {
#pragma unroll
        for (int k = 0; k < QK; ++k) nv[k] = *reinterpret_cast<const f4 *>(p.norm_w + (k0 + k) * 256 + lane * 4);
    }
    f4 wv[NR][IN4];
    f4 wu[NR][IN4];
    u2 bv[NR][IN4];
    u2 bu[NR][IN4];
    float yv[NR];   // kEpiAccum: the residual rows, loaded with the weights so that the store needs no load
    auto load_rows = [&](int o0) {
        if constexpr (EPI == kEpiAccum) {
#pragma unroll
            for (int r = 0; r < NR; ++r) yv[r] = p.res[min(o0 + r, p.out_dim - 1)];
        }
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int64_t o = min(o0 + r, p.out_dim - 1);
            if constexpr (B16) {
                const uint16_t * wr = static_cast<const uint16_t *>(p.W) + o * in + lane * 4;
#pragma unroll
                for (int k = 0; k < IN4; ++k) {
                    bv[r][k] = __builtin_nontemporal_load(reinterpret_cast<const u2 *>(wr + k * 256));
                }
                if constexpr (EPI == kEpiSwiglu) {
                    const uint16_t * wur = static_cast<const uint16_t *>(p.W) + (o + p.out_dim) * in + lane * 4;
#pragma unroll
                    for (int k = 0; k < IN4; ++k) {
                        bu[r][k] = __builtin_nontemporal_load(reinterpret_cast<const u2 *>(wur + k * 256));
                    }
                }
            } else {
                const float * wr = static_cast<const float *>(p.W) + o * in + lane * 4;
#pragma unroll
                for (int k = 0; k < IN4; ++k) {
                    wv[r][k] = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(wr + k * 256));
                }
                if constexpr (EPI == kEpiSwiglu) {
                    const float * wur = static_cast<const float *>(p.W) + (o + p.out_dim) * in + lane * 4;
#pragma unroll
                    for (int k = 0; k < IN4; ++k) {
                        wu[r][k] = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(wur + k * 256));
                    }
                }
            }
        }
    };
    int o0 = gw * NR;
    // every wave takes part in the staging barriers; a wave past the last row loads the last row's
    // weights (load_rows clamps) and stores nothing
    asm volatile("" ::: "memory");   // x and the norm weight are issued before the weight rows
    load_rows(o0);
    // every load above is issued before the norm arithmetic: the empty asm orders the loads before it
    // (memory clobber) and the arithmetic after it (it redefines x), otherwise the scheduler hoists the
    // reduction, and its wait for x, above the weight loads
#pragma unroll
    for (int k = 0; k < QK; ++k) asm volatile("" : "+v"(xv[k]) : : "memory");
    if constexpr (PRENORM) {
        // rms_norm_row (text-decoder.cpp:542-557): squares in double, float scale, (x * scale) * w; the
        // squares are summed per wave quarter in double, the four quarters in a fixed order
        __shared__ double s_ss[4];
        __shared__ f4 s_x[IN4 * kWave];
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < QK; ++k) {
            ss += static_cast<double>(xv[k].x) * xv[k].x + static_cast<double>(xv[k].y) * xv[k].y +
                  static_cast<double>(xv[k].z) * xv[k].z + static_cast<double>(xv[k].w) * xv[k].w;
        }
        ss = wave_sum_d_lane63(ss);
        if (lane == kWave - 1) s_ss[wave] = ss;
        __syncthreads();
        const double tot = (s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3]);
        const float scale = 1.0f / sqrtf(static_cast<float>(tot / static_cast<double>(p.in_dim)) + p.eps);
#pragma unroll
        for (int k = 0; k < QK; ++k) {
            f4 v;
            v.x = xv[k].x * scale * nv[k].x;
            v.y = xv[k].y * scale * nv[k].y;
            v.z = xv[k].z * scale * nv[k].z;
            v.w = xv[k].w * scale * nv[k].w;
            s_x[(k0 + k) * kWave + lane] = v;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < IN4; ++k) xv[k] = s_x[k * kWave + lane];
    } else {
        __shared__ f4 s_x[IN4 * kWave];
#pragma unroll
        for (int k = 0; k < QK; ++k) s_x[(k0 + k) * kWave + lane] = xv[k];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < IN4; ++k) xv[k] = s_x[k * kWave + lane];
    }
    for (;;) {
        float acc[NR];
        float accu[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) { acc[r] = 0.0f; accu[r] = 0.0f; }
#pragma unroll
        for (int r = 0; r < NR; ++r) {
#pragma unroll
            for (int k = 0; k < IN4; ++k) {
                if constexpr (B16) {
                    acc[r] = dot4(widen_bf16x4(bv[r][k]), xv[k], acc[r]);
                    if constexpr (EPI == kEpiSwiglu) accu[r] = dot4(widen_bf16x4(bu[r][k]), xv[k], accu[r]);
                } else {
                    acc[r] = dot4(wv[r][k], xv[k], acc[r]);
                    if constexpr (EPI == kEpiSwiglu) accu[r] = dot4(wu[r][k], xv[k], accu[r]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const float a = wave_sum_lane63(acc[r]);
            float u = 0.0f;
            if constexpr (EPI == kEpiSwiglu) u = wave_sum_lane63(accu[r]);
            const int o = o0 + r;
            if (lane == kWave - 1 && o < p.out_dim) {
                if constexpr (EPI == kEpiStore) st_f<COH>(p.y + o, a);
                else if constexpr (EPI == kEpiAccum) st_f<COH>(p.y + o, yv[r] + a);
                else st_f<COH>(p.y + o, (a / (1.0f + expf(-a))) * u);   // silu(gate) * up (text-decoder.cpp:602)
            }
        }
        o0 += nw * NR;
        if (o0 >= p.out_dim) break;
        load_rows(o0);
    }
}

}  // namespace
}  // namespace qa
