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
// columns.
//
// Exact GGML softmax needs the row max and sum before any PV, so the key tiles are walked twice:
//   pass 1  S^T, a running max per lane and the sum of exp(s - max): 16 terms in f32 per tile and
//           lane, carried across tiles in double and rescaled when the lane's max grows; the 4 lanes
//           of a query column are combined once at the end;
//   pass 2  S^T again, p = f16(exp(s - M) * (float)(1 / sum)), O^T += V^T P^T.
// exp(x * scale - m) is evaluated as exp2(x * (scale log2 e) - m (scale log2 e)): one FMA and one
// v_exp_f32 per score.  Its rounding differs from a library expf by a few f32 ulps, far below the f16
// resolution of p (the reference's own CPU softmax uses a vectorised exp approximation as well).
// Only the diagonal tiles (keys past the first query of the workgroup) are masked; every other tile
// takes an unmasked path.
// P^T goes from the accumulator registers straight into the B operand of the PV MFMA: the PV k-index
// e of lane group j is mapped to key (e / 4) * 16 + j * 4 + e % 4 of the 32-key step, which is
// exactly the set of keys that lane already holds; V^T is read from LDS with the same mapping.
//
// LDS: two buffers of the K tile (row-major, 144-half rows) and of V^T (dims x keys in PV order,
// 80-half rows): one barrier per tile; the next tile's global loads are in registers while the current
// one is computed.  Both operands are read as 16-byte rows at conflict-free strides.  V^T is written as
// 4 keys x 1 dim per 8-byte store, transposed in registers from 4 rows of 8 dims.
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
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kBQ = 64;     // query tokens per workgroup
constexpr int kBK = 64;     // keys per tile
// Row strides: a 16-byte LDS read by 16 lanes of consecutive rows is conflict-free on gfx950 when the
// stride in dwords is 8 mod 16 (measured: 80, 112, 144 halfs conflict-free; 72, 88, 96, 136 halfs
// lose ~half the LDS cycles to bank conflicts).
constexpr int kKS = 144;    // K tile row stride (halfs): 128 dims + 16
constexpr int kVS = 80;     // V^T tile row stride (halfs): 64 keys + 16
constexpr float kLog2e = 1.4426950408889634f;

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

// Global -> register staging of one tile.  K: thread t loads 16-byte slices idx = it * 256 + t
// (row idx / 16, slice idx % 16).  V: thread t loads slice dg = 4 * wave + lane / 16 of the 4 rows
// 4 kq .. 4 kq + 3 with kq = lane % 16, which it writes transposed.  Rows past the end re-read the last
// row (masked keys get p = 0; no branch splits the loads).
struct TileRegs {
    u4 k[4];
    u4 v[4];
};

__device__ inline void load_tile(const _Float16 * kh, const _Float16 * vh, int kt, int kend, bool with_v,
                                 TileRegs & r) {
    const int t = threadIdx.x;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = it * 256 + t;
        const int row = min(kt * kBK + (idx >> 4), kend - 1);
        r.k[it] = *reinterpret_cast<const u4 *>(kh + static_cast<int64_t>(row) * kHeadDim + (idx & 15) * 8);
    }
    if (!with_v) return;
    const int kq = t & 15, dg = t >> 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int row = min(kt * kBK + kq * 4 + e, kend - 1);
        r.v[e] = *reinterpret_cast<const u4 *>(vh + static_cast<int64_t>(row) * kHeadDim + dg * 8);
    }
}

__device__ inline uint32_t lo_pair(uint32_t a, uint32_t b) { return (a & 0xffffu) | (b << 16); }
__device__ inline uint32_t hi_pair(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xffff0000u); }

__device__ inline void store_tile(const TileRegs & r, _Float16 * sK, _Float16 * sV, bool with_v) {
    const int t = threadIdx.x;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = it * 256 + t;
        *reinterpret_cast<u4 *>(sK + (idx >> 4) * kKS + (idx & 15) * 8) = r.k[it];
    }
    if (!with_v) return;
    const int kq = t & 15, dg = t >> 4;
    // V^T columns are keys in PV order: key j sits at column (j / 32) * 32 + ((j % 16) / 4) * 8 +
    // ((j / 16) % 2) * 4 + j % 4, so the 8 keys one lane multiplies in a 32-key step (4 from each 16-key
    // block) are 8 consecutive halfs: one 16-byte read.  Keys 4 kq .. 4 kq + 3 stay adjacent.
    const int col = (kq >> 3) * 32 + (kq & 3) * 8 + ((kq >> 2) & 1) * 4;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        // dims 2w and 2w + 1 of the slice, keys 4 kq .. 4 kq + 3
        const uint2 even = make_uint2(lo_pair(r.v[0][w], r.v[1][w]), lo_pair(r.v[2][w], r.v[3][w]));
        const uint2 odd = make_uint2(hi_pair(r.v[0][w], r.v[1][w]), hi_pair(r.v[2][w], r.v[3][w]));
        *reinterpret_cast<uint2 *>(sV + (dg * 8 + 2 * w) * kVS + col) = even;
        *reinterpret_cast<uint2 *>(sV + (dg * 8 + 2 * w + 1) * kVS + col) = odd;
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

// Masks the keys of a diagonal tile: key j of query column cb is attended iff j <= lim[cb].
__device__ inline void mask_tile(f4 (&S)[4][2], const int (&lim)[2], int kt, int g4) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = kt * kBK + kb * 16 + g4 * 4 + i;
                if (j > lim[cb]) S[kb][cb][i] = -INFINITY;
            }
        }
    }
}

// Pass-1 update of one lane's running max m (raw score units) and double sum of exp(s - m).
__device__ inline void stats_update(const f4 (&S)[4][2], int cb, float c, float & m, double & sum) {
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, S[kb][cb][i]);
    }
    const float mn = fmaxf(m, tmax);
    if (mn == -INFINITY) return;                 // every key so far masked for this lane
    const float mc = mn * c;
    float part = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) part += __builtin_amdgcn_exp2f(fmaf(S[kb][cb][i], c, -mc));
    }
    // exp2(-inf) = 0 when the lane had nothing before this tile
    const float f = __builtin_amdgcn_exp2f(fmaf(m, c, -mc));
    sum = sum * static_cast<double>(f) + static_cast<double>(part);
    m = mn;
}

__device__ inline void pv_tile(const f4 (&S)[4][2], const _Float16 * sV, const float (&mc)[2], const float (&r)[2],
                               float c, int c16, int g4, f4 (&O)[8][2]) {
    // P^T fragments: pf[cb][ksv] element e <-> key (2 ksv + e / 4) * 16 + g4 * 4 + e % 4
    h8 pf[2][2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float pv = __builtin_amdgcn_exp2f(fmaf(S[kb][cb][i], c, -mc[cb])) * r[cb];
                pf[cb][kb >> 1][(kb & 1) * 4 + i] = static_cast<_Float16>(pv);
            }
        }
    }
#pragma unroll
    for (int ksv = 0; ksv < 2; ++ksv) {
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            const h8 a = *reinterpret_cast<const h8 *>(sV + (db * 16 + c16) * kVS + ksv * 32 + g4 * 8);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                O[db][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pf[cb][ksv], O[db][cb], 0, 0, 0);
            }
        }
    }
}

__global__ __launch_bounds__(256, 2) void prefill_mfma_kernel(MfmaParams p) {
    __shared__ __attribute__((aligned(16))) _Float16 sK[2][kBK * kKS];
    __shared__ __attribute__((aligned(16))) _Float16 sV[2][kHeadDim * kVS];

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
    // tiles below kt_full hold only keys <= n_past + t0, attended by every query of the workgroup
    const int kt_full = min((p.n_past + t0 + 1) / kBK, n_kt);
    const _Float16 * kh = p.k + g * p.head_stride;
    const _Float16 * vh = p.v + g * p.head_stride;
    const float c = p.scale * kLog2e;

    // query columns of this lane and their causal key limits
    int tq[2], lim[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        tq[cb] = tw + cb * 16 + c16;
        lim[cb] = tq[cb] < p.n_tokens ? p.n_past + tq[cb] : -1;   // keys j <= lim are attended
    }

    // Q fragments, the B operand of S^T: lane holds query column c16 and 8 dims of each 32-dim step,
    // rounded to f16 (GGML's conversion of src1 for an f16 src0); absent tokens are zero
    h8 qf[2][4];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const int tqc = min(tq[cb], p.n_tokens - 1);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const float * qp = p.q + static_cast<int64_t>(tqc) * p.q_stride + h * kHeadDim + ks * 32 + g4 * 8;
            const float4 a = *reinterpret_cast<const float4 *>(qp);
            const float4 b = *reinterpret_cast<const float4 *>(qp + 4);
            const bool ok = tq[cb] < p.n_tokens;
            qf[cb][ks] = h8{static_cast<_Float16>(ok ? a.x : 0.f), static_cast<_Float16>(ok ? a.y : 0.f),
                            static_cast<_Float16>(ok ? a.z : 0.f), static_cast<_Float16>(ok ? a.w : 0.f),
                            static_cast<_Float16>(ok ? b.x : 0.f), static_cast<_Float16>(ok ? b.y : 0.f),
                            static_cast<_Float16>(ok ? b.z : 0.f), static_cast<_Float16>(ok ? b.w : 0.f)};
        }
    }

    // ---------------------------------------------------------------- pass 1: max and sum
    float m[2] = {-INFINITY, -INFINITY};
    double sum[2] = {0.0, 0.0};
    TileRegs regs;
    load_tile(kh, vh, 0, kend, false, regs);
    store_tile(regs, sK[0], sV[0], false);
    if (n_kt > 1) load_tile(kh, vh, 1, kend, false, regs);
    __syncthreads();
    for (int kt = 0; kt < n_kt; ++kt) {
        f4 S[4][2];
        scores_tile(sK[kt & 1], qf, c16, g4, S);
        if (kt >= kt_full) mask_tile(S, lim, kt, g4);
        stats_update(S, 0, c, m[0], sum[0]);
        stats_update(S, 1, c, m[1], sum[1]);
        if (kt + 1 < n_kt) {
            store_tile(regs, sK[(kt + 1) & 1], sV[(kt + 1) & 1], false);
            if (kt + 2 < n_kt) load_tile(kh, vh, kt + 2, kend, false, regs);
        }
        __syncthreads();
    }
    // combine the 4 lanes of each query column (lane bits 4, 5)
    float mc[2], r[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        float M = fmaxf(m[cb], __shfl_xor(m[cb], 16, kWave));
        M = fmaxf(M, __shfl_xor(M, 32, kWave));
        double s = M == -INFINITY ? 0.0 : sum[cb] * static_cast<double>(__builtin_amdgcn_exp2f((m[cb] - M) * c));
        s += __shfl_xor(s, 16, kWave);
        s += __shfl_xor(s, 32, kWave);
        mc[cb] = M == -INFINITY ? 0.0f : M * c;
        r[cb] = s > 0.0 ? static_cast<float>(1.0 / s) : 0.0f;
    }

    // ---------------------------------------------------------------- pass 2: p and PV
    f4 O[8][2];
#pragma unroll
    for (int db = 0; db < 8; ++db) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) O[db][cb] = f4{0.f, 0.f, 0.f, 0.f};
    }
    load_tile(kh, vh, 0, kend, true, regs);
    store_tile(regs, sK[0], sV[0], true);
    if (n_kt > 1) load_tile(kh, vh, 1, kend, true, regs);
    __syncthreads();
    for (int kt = 0; kt < n_kt; ++kt) {
        f4 S[4][2];
        scores_tile(sK[kt & 1], qf, c16, g4, S);
        if (kt >= kt_full) mask_tile(S, lim, kt, g4);
        pv_tile(S, sV[kt & 1], mc, r, c, c16, g4, O);
        if (kt + 1 < n_kt) {
            store_tile(regs, sK[(kt + 1) & 1], sV[(kt + 1) & 1], true);
            if (kt + 2 < n_kt) load_tile(kh, vh, kt + 2, kend, true, regs);
        }
        __syncthreads();
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
