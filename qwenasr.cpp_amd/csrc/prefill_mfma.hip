// Causal prefill attention on CDNA4 f16 MFMA (v_mfma_f32_16x16x32_f16), for f16 KV caches.
//
// Replaces the prefill half of the cached layer graph (text-decoder.cpp:435-463 with T > 1 and the
// dense mask of 1729-1735): scores = mul_mat(K, q), soft_max_ext(scores, mask, 1/sqrt(d)),
// out = mul_mat(cont(V^T), p).  With f16 K/V the reference's GGML arithmetic rounds q to f16 before
// QK^T and the normalised probabilities to f16 before PV; both are exactly the f16 operands the MFMA
// takes, with f32 accumulation.
//
// Tiling.  A workgroup (4 waves) owns 64 query tokens of one stream and both query heads of one KV
// head: 128 query columns, every K/V byte of the head shared by both heads.  Wave w takes head
// 2g + w/2 and tokens [32 (w & 1), +32).  Per 64-key tile a wave computes S^T = K Q^T (keys x queries,
// 16x16 blocks, head dim in 4 steps of 32), so after the MFMA each lane holds 16 keys of 2 query
// columns and the softmax statistics of a query are a reduction over 4 lanes (xor 16, 32).
//
// Exact GGML softmax needs the row max and sum before any PV, so the key tiles are walked twice:
//   pass 1  S^T, running max, and the sum of expf(s - max) in double, rescaled when the max grows;
//   pass 2  S^T again, p = f16(expf(s - M) * (float)(1 / sum)), O^T += V^T P^T.
// P^T goes from the accumulator registers straight into the B operand of the PV MFMA: the PV k-index
// e of lane group j is mapped to key (e / 4) * 16 + j * 4 + e % 4 of the 32-key step, which is
// exactly the set of keys that lane already holds; V^T is read from LDS with the same mapping.
//
// LDS: the K tile is stored row-major with a 136-half row stride and V transposed (V^T, dims x keys)
// with a 68-half stride, so the 16-byte K reads and 8-byte V^T reads of 16 lanes hit distinct banks.
// The next tile's global loads are issued before the current tile's MFMAs (register double buffer).
// Block mapping: blockIdx.x = (n_qt - 1 - tile) * n_kv + kv_head, so consecutive workgroups (dispatched
// round-robin over the 8 XCDs) are the 8 KV heads of one tile: every tile of one KV head lands on the
// same XCD, whose L2 then holds that head's K/V (2 MB at 3913 positions) for all of its tiles; the
// heaviest (last, causally longest) tiles start first.
#include "ops.hpp"

#include <cmath>

namespace qa {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kBQ = 64;     // query tokens per workgroup
constexpr int kBK = 64;     // keys per tile
constexpr int kKS = 136;    // K tile row stride (halfs)
constexpr int kVS = 68;     // V^T tile row stride (halfs)

struct MfmaParams {
    const float * q;          // [T][q_stride], token t of the call
    const _Float16 * k;       // this layer/stream's K rows, head 0 position 0
    const _Float16 * v;
    float * out;              // [T][q_stride]
    int64_t head_stride;      // elements between KV heads (max_seq * 128)
    int32_t q_stride;
    int32_t n_past, n_tokens, n_kv, n_qt;
    float scale;
};

struct TileRegs {
    uint4 k[4];               // 4 x 16 B of the K tile
    uint4 v[2][2];            // 2 key pairs x 2 keys x 16 B of the V tile
};

__device__ inline void load_tile(const MfmaParams & p, const _Float16 * kh, const _Float16 * vh, int kt, int kend,
                                 TileRegs & r) {
    const int t = threadIdx.x;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = it * 256 + t;
        const int row = idx >> 4, c = idx & 15;
        const int j = kt * kBK + row;
        r.k[it] = j < kend ? *reinterpret_cast<const uint4 *>(kh + static_cast<int64_t>(j) * kHeadDim + c * 8)
                           : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int idx = it * 256 + t;
        const int kp = idx >> 4, dg = idx & 15;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int j = kt * kBK + 2 * kp + e;
            r.v[it][e] = j < kend ? *reinterpret_cast<const uint4 *>(vh + static_cast<int64_t>(j) * kHeadDim + dg * 8)
                                  : make_uint4(0, 0, 0, 0);
        }
    }
}

__device__ inline void store_tile(const TileRegs & r, _Float16 * sK, _Float16 * sV, bool with_v) {
    const int t = threadIdx.x;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = it * 256 + t;
        const int row = idx >> 4, c = idx & 15;
        *reinterpret_cast<uint4 *>(sK + row * kKS + c * 8) = r.k[it];
    }
    if (!with_v) return;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int idx = it * 256 + t;
        const int kp = idx >> 4, dg = idx & 15;
        const h8 a = __builtin_bit_cast(h8, r.v[it][0]);
        const h8 b = __builtin_bit_cast(h8, r.v[it][1]);
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            h2 pair;
            pair[0] = a[d];
            pair[1] = b[d];
            *reinterpret_cast<h2 *>(sV + (dg * 8 + d) * kVS + 2 * kp) = pair;
        }
    }
}

// S^T tile of this wave: S[kb][cb] = 16 keys (kb) x 16 queries (cb).
__device__ inline void scores_tile(const _Float16 * sK, const h8 (&qf)[2][4], int c16, int g4, f4 (&S)[4][2]) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) S[kb][cb] = f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const h8 a = *reinterpret_cast<const h8 *>(sK + (kb * 16 + c16) * kKS + ks * 32 + g4 * 8);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                S[kb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[cb][ks], S[kb][cb], 0, 0, 0);
            }
        }
    }
}

__global__ __launch_bounds__(256) void prefill_mfma_kernel(MfmaParams p) {
    __shared__ __attribute__((aligned(16))) _Float16 sK[kBK * kKS];
    __shared__ __attribute__((aligned(16))) _Float16 sV[kHeadDim * kVS];

    const int g = static_cast<int>(blockIdx.x) % p.n_kv;
    const int qt = p.n_qt - 1 - static_cast<int>(blockIdx.x) / p.n_kv;
    const int t0 = qt * kBQ;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int hh = wave >> 1;
    const int h = g * 2 + hh;
    const int tw = t0 + (wave & 1) * 32;
    const int c16 = lane & 15;
    const int g4 = lane >> 4;
    const int L_total = p.n_past + p.n_tokens;
    const int kend = min(L_total, p.n_past + min(t0 + kBQ, p.n_tokens));
    const int n_kt = (kend + kBK - 1) / kBK;
    const _Float16 * kh = p.k + g * p.head_stride;
    const _Float16 * vh = p.v + g * p.head_stride;

    // query columns of this lane and their causal key limits
    int tq[2], lim[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        tq[cb] = tw + cb * 16 + c16;
        lim[cb] = tq[cb] < p.n_tokens ? p.n_past + tq[cb] : -1;   // keys j <= lim are attended
    }

    // Q fragments, the B operand of S^T: lane holds query column c16 and 8 dims of each 32-dim step,
    // rounded to f16 (GGML's conversion of src1 for an f16 src0)
    h8 qf[2][4];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if (tq[cb] < p.n_tokens) {
                const float * qp = p.q + static_cast<int64_t>(tq[cb]) * p.q_stride + h * kHeadDim + ks * 32 + g4 * 8;
                const float4 a = *reinterpret_cast<const float4 *>(qp);
                const float4 b = *reinterpret_cast<const float4 *>(qp + 4);
                qf[cb][ks] = h8{static_cast<_Float16>(a.x), static_cast<_Float16>(a.y), static_cast<_Float16>(a.z),
                                static_cast<_Float16>(a.w), static_cast<_Float16>(b.x), static_cast<_Float16>(b.y),
                                static_cast<_Float16>(b.z), static_cast<_Float16>(b.w)};
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) qf[cb][ks][e] = static_cast<_Float16>(0.0f);
            }
        }
    }

    // ---------------------------------------------------------------- pass 1: max and sum
    float m[2] = {-INFINITY, -INFINITY};
    double sum[2] = {0.0, 0.0};
    TileRegs regs;
    if (n_kt > 0) load_tile(p, kh, vh, 0, kend, regs);
    for (int kt = 0; kt < n_kt; ++kt) {
        __syncthreads();
        store_tile(regs, sK, sV, false);
        __syncthreads();
        if (kt + 1 < n_kt) load_tile(p, kh, vh, kt + 1, kend, regs);
        f4 S[4][2];
        scores_tile(sK, qf, c16, g4, S);
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            float x[16];
            float tmax = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int j = kt * kBK + kb * 16 + g4 * 4 + i;
                    const float s = S[kb][cb][i] * p.scale;
                    x[kb * 4 + i] = j <= lim[cb] ? s : -INFINITY;
                    tmax = fmaxf(tmax, x[kb * 4 + i]);
                }
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
            const float mn = fmaxf(m[cb], tmax);
            if (mn == -INFINITY) continue;            // nothing attended yet for this column
            if (mn > m[cb]) {
                sum[cb] = m[cb] == -INFINITY ? 0.0 : sum[cb] * exp(static_cast<double>(m[cb]) - static_cast<double>(mn));
                m[cb] = mn;
            }
            double e = 0.0;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                if (x[k] != -INFINITY) e += static_cast<double>(expf(x[k] - mn));
            }
            sum[cb] += e;
        }
    }
    float r[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        double s = sum[cb];
        s += __shfl_xor(s, 16, kWave);
        s += __shfl_xor(s, 32, kWave);
        r[cb] = s > 0.0 ? static_cast<float>(1.0 / s) : 0.0f;
    }

    // ---------------------------------------------------------------- pass 2: p and PV
    f4 O[8][2];
#pragma unroll
    for (int db = 0; db < 8; ++db) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) O[db][cb] = f4{0.f, 0.f, 0.f, 0.f};
    }
    if (n_kt > 0) load_tile(p, kh, vh, 0, kend, regs);
    for (int kt = 0; kt < n_kt; ++kt) {
        __syncthreads();
        store_tile(regs, sK, sV, true);
        __syncthreads();
        if (kt + 1 < n_kt) load_tile(p, kh, vh, kt + 1, kend, regs);
        f4 S[4][2];
        scores_tile(sK, qf, c16, g4, S);
        // P^T fragments: pf[cb][ksv] element e <-> key (2 ksv + e / 4) * 16 + g4 * 4 + e % 4
        h8 pf[2][2];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int j = kt * kBK + kb * 16 + g4 * 4 + i;
                    const float s = S[kb][cb][i] * p.scale;
                    const float pv = j <= lim[cb] ? expf(s - m[cb]) * r[cb] : 0.0f;
                    pf[cb][kb >> 1][(kb & 1) * 4 + i] = static_cast<_Float16>(pv);
                }
            }
        }
#pragma unroll
        for (int ksv = 0; ksv < 2; ++ksv) {
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                const _Float16 * vr = sV + (db * 16 + c16) * kVS + (2 * ksv) * 16 + g4 * 4;
                const h4 lo = *reinterpret_cast<const h4 *>(vr);
                const h4 hi = *reinterpret_cast<const h4 *>(vr + 16);
                const h8 a = h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) {
                    O[db][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pf[cb][ksv], O[db][cb], 0, 0, 0);
                }
            }
        }
    }

    // O^T: lane holds dims db * 16 + g4 * 4 + i of query column c16 of block cb
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        if (tq[cb] >= p.n_tokens) continue;
        float * op = p.out + static_cast<int64_t>(tq[cb]) * p.q_stride + h * kHeadDim + g4 * 4;
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            *reinterpret_cast<float4 *>(op + db * 16) = make_float4(O[db][cb][0], O[db][cb][1], O[db][cb][2], O[db][cb][3]);
        }
    }
}

}  // namespace

int prefill_mfma_launch(const float * q, int32_t q_stride, const void * k, const void * v, int64_t head_stride,
                        int32_t n_past, int32_t n_tokens, int32_t n_kv, float scale, float * out, hipStream_t stream) {
    MfmaParams p{};
    p.q = q;
    p.k = static_cast<const _Float16 *>(k);
    p.v = static_cast<const _Float16 *>(v);
    p.out = out;
    p.head_stride = head_stride;
    p.q_stride = q_stride;
    p.n_past = n_past;
    p.n_tokens = n_tokens;
    p.n_kv = n_kv;
    p.n_qt = (n_tokens + kBQ - 1) / kBQ;
    p.scale = scale;
    const int64_t blocks = static_cast<int64_t>(p.n_qt) * n_kv;
    if (blocks <= 0) return QA_OK;
    hipLaunchKernelGGL(prefill_mfma_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p);
    QA_LAUNCH_CHECK("prefill_mfma_kernel");
    return QA_OK;
}

}  // namespace qa
