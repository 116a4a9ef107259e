// Prefill projections on bf16-exact weights, gfx950 (bf16 MFMA, v_mfma_f32_32x32x16_bf16).
//
// Replaces linear_ggml with PREC_F32 (text-decoder.cpp:83-90) for T > 32 rows when the f32 weights are
// bf16-exact (their low 16 bits are zero, as in every checkpoint converted from the released bf16 weights,
// convert.py:386-387).  Each input row x arrives split into three bf16 parts, x = hi + mid + lo exactly
// (split3.hpp), so
//     Y[t][n] (+)= sum_p sum_k Xs[t][p K + k] W[n][k]
// multiplies every weight by every part exactly in f32 and sums in f32: f32 products and f32 sums, as the
// reference's f32 GEMM, in another order.  The kernel reads the one bf16 copy of W and uses each W tile for
// the three parts (a library GEMM would need the rows tripled, [W W W], to see the sum as one product).
//
// Tiling.  A workgroup (8 waves) owns 128 token rows x 256 output columns; each wave 64 x 64 (2 x 2 MFMA
// tiles of 32 x 32).  A stage holds 64 k of the tile: the 3 x 128 Xs rows and 256 W rows, 128 B each,
// 80 KB of LDS, loaded with global_load_lds_dwordx4 straight into LDS (no register staging).  LDS blocks are
// 8 rows x 128 B; lane l of a load instruction fills 16-byte slot l % 8 of row l / 8, so 8 lanes cover one
// whole 128-byte line (full-line requests: 64-byte half lines measured 25% slower), and the slot holds the
// row's global chunk (l % 8) ^ (l / 8): an MFMA operand read (32 rows x 16 bytes, chunk c of row r in slot
// c ^ (r % 8)) then hits 8 distinct 16-byte bank groups per 8 lanes.
// Two schedules, chosen by the grid size:
//   RING 2: two LDS stages (160 KB, one workgroup per CU); stage s + 1 loads while stage s computes.  For
//           grids of about one workgroup per CU (o, down at T = 3913: 248 workgroups) and for the
//           accumulating epilogue.
//   RING 1: one stage (80 KB) and two workgroups per CU, each loading then computing; the two workgroups
//           drift into alternating phases, so one computes while the other loads.  For larger grids
//           (q|k|v 496, gate|up 1488 workgroups): 149 against 170 us (q|k|v), 453 against 508 us (gate|up).
// Workgroup i runs on XCD i % 8: when the output columns split into a multiple of 8 tiles, XCD x takes
// column tiles [x n / 8, (x + 1) n / 8) for every token tile, walked token-major, so that the workgroups
// resident on one XCD share their W and Xs tiles in its L2.
//
// Epilogues: store Y; accumulate into Y (the residual adds of o and down, text-decoder.cpp:465, 493);
// SwiGLU (text-decoder.cpp:602): W holds [gate rows; up rows], each workgroup loads 128 gate rows and the
// 128 matching up rows (wave tile 32 gate + 32 up columns, so both values of an output sit in one lane),
// and writes silu(gate) * up as the three-part split that the down projection reads -- the [T][2 I] f32
// gate|up output never goes to memory.
#include "ops.hpp"
#include "split3.hpp"

#include <cmath>

namespace qa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kBM = 128;                                // token rows per workgroup
constexpr int kBN = 256;                                // W rows per workgroup
constexpr int kBK = 64;                                 // k per stage
constexpr int kThreads = 512;
constexpr int kXsBlocks = 3 * kBM / 8;                  // 1 KB LDS blocks (8 rows x 128 B) per stage
constexpr int kWBlocks = kBN / 8;
constexpr int kStage = (kXsBlocks + kWBlocks) * 1024;   // 80 KB
constexpr int kLoadsPerWave = (kXsBlocks + kWBlocks) / 8;
static_assert((kXsBlocks + kWBlocks) % 8 == 0, "load instructions split evenly over the waves");

enum { kS3Store = 0, kS3Accumulate = 1, kS3Swiglu = 2 };

struct Split3Params {
    const uint16_t * W;      // [rows of W][K] bf16 bits
    const uint16_t * Xs;     // [M][3 K] bf16 bits
    float * Y;               // [M][N] f32 (store, accumulate)
    uint16_t * act;          // SwiGLU: [M][3 N] split of silu(gate) * up
    int32_t M, N, K;         // N output columns (SwiGLU: W has 2 N rows, gate rows then up rows)
    int32_t m_tiles, n_tiles;
};

__device__ inline void wait_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int RING, int EPI>
__global__ __launch_bounds__(kThreads) void gemm_split3_kernel(Split3Params p) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(1024))) unsigned char lds[RING * kStage];
    constexpr int kCols = EPI == kS3Swiglu ? kBN / 2 : kBN;   // output columns per workgroup
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    int mt, nt;
    if (p.n_tiles % 8 == 0) {
        const int per = p.n_tiles / 8, xcd = blockIdx.x % 8, j = blockIdx.x / 8;
        mt = j / per;
        nt = xcd * per + j % per;
    } else {
        mt = blockIdx.x % p.m_tiles;
        nt = blockIdx.x / p.m_tiles;
    }
    const int m0 = mt * kBM, c0 = nt * kCols;
    const int64_t ldx = 3 * static_cast<int64_t>(p.K);

    // source rows of this wave's load instructions (block wave + 8 u of a stage)
    const int lrow = lane >> 3, lchunk = (lane & 7) ^ (lane >> 3);
    const uint16_t * src[kLoadsPerWave];
#pragma unroll
    for (int u = 0; u < kLoadsPerWave; ++u) {
        const int blk = wave + 8 * u;
        if (blk < kXsBlocks) {
            const int row = blk * 8 + lrow;                  // part p: rows p kBM .. p kBM + kBM - 1
            const int part = row / kBM, t = row % kBM;
            src[u] = p.Xs + min(m0 + t, p.M - 1) * ldx + static_cast<int64_t>(part) * p.K + lchunk * 8;
        } else {
            const int f = (blk - kXsBlocks) * 8 + lrow;      // LDS W row 0..255: tile f / 32, row f % 32
            int64_t wrow;
            if (EPI == kS3Swiglu) {
                // tile 2 q: gate rows c0 + 32 q + 0..31; tile 2 q + 1: the matching up rows
                const int q = f >> 6, up = (f >> 5) & 1, r = f & 31;
                wrow = static_cast<int64_t>(up) * p.N + c0 + 32 * q + r;
            } else {
                wrow = c0 + f;
            }
            src[u] = p.W + wrow * p.K + lchunk * 8;
        }
    }
    auto issue = [&](int s) {
        unsigned char * st = lds + (s % RING) * kStage;
        const int k0 = s * kBK;
#pragma unroll
        for (int u = 0; u < kLoadsPerWave; ++u)
            __builtin_amdgcn_global_load_lds(src[u] + k0, st + (wave + 8 * u) * 1024, 16, 0, 0);
    };

    // wave (wt, wf): tokens 64 wt .. + 63 (Xs tiles 2 wt, 2 wt + 1), W tiles 2 wf, 2 wf + 1
    const int wt = wave & 1, wf = wave >> 1;
    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v16f{};
    const int rr = lane & 31;
    auto rdo = [&](int b) {   // operand row rr, chunk 2 b + lane / 32 of a 32-row tile (4 blocks)
        return 1024 * (rr >> 3) + 128 * (rr & 7) + 16 * ((2 * b + (lane >> 5)) ^ (rr & 7));
    };
    auto compute = [&](const unsigned char * buf) {
#pragma unroll
        for (int b = 0; b < kBK / 16; ++b) {
            bf16x8 bw[2];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
                bw[jj] = *reinterpret_cast<const bf16x8 *>(buf + (kXsBlocks + 4 * (2 * wf + jj)) * 1024 + rdo(b));
#pragma unroll
            for (int part = 0; part < 3; ++part) {
                bf16x8 ax[2];
#pragma unroll
                for (int ii = 0; ii < 2; ++ii)
                    ax[ii] = *reinterpret_cast<const bf16x8 *>(buf + (16 * part + 4 * (2 * wt + ii)) * 1024 + rdo(b));
#pragma unroll
                for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                    for (int jj = 0; jj < 2; ++jj)
                        acc[ii][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ax[ii], bw[jj], acc[ii][jj], 0, 0, 0);
            }
        }
    };
    const int ns = p.K / kBK;
    if constexpr (RING == 1) {
        for (int s = 0; s < ns; ++s) {
            issue(s);
            wait_loads();
            __syncthreads();
            compute(lds);
            __syncthreads();
        }
    } else {
        issue(0);
        for (int s = 0; s < ns; ++s) {
            wait_loads();                  // stage s (the only loads in flight)
            __syncthreads();               // every wave's part of stage s; compute(s - 1) done everywhere
            if (s + 1 < ns) issue(s + 1);  // into the buffer compute(s - 1) read
            compute(lds + (s & 1) * kStage);
        }
    }

    // D[token row][column]: column lane % 32, row 8 (e / 4) + 4 (lane / 32) + e % 4 of the 32 x 32 tile
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const int tb = m0 + 32 * (2 * wt + ii) + 4 * (lane >> 5);
        if constexpr (EPI == kS3Swiglu) {
            const int col = c0 + 32 * wf + rr;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int t = tb + 8 * (e >> 2) + (e & 3);
                const float g = acc[ii][0][e], u = acc[ii][1][e];
                if (t < p.M) store_split3(p.act + static_cast<int64_t>(t) * 3 * p.N + col, p.N, (g / (1.0f + expf(-g))) * u);
            }
        } else {
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int col = c0 + 32 * (2 * wf + jj) + rr;
                if constexpr (EPI == kS3Accumulate) {
                    // old values 8 at a time, all 8 in flight together (rows past M re-read row M - 1)
#pragma unroll
                    for (int h = 0; h < 16; h += 8) {
                        float old[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            old[e] = p.Y[static_cast<int64_t>(min(tb + 8 * ((h + e) >> 2) + (e & 3), p.M - 1)) * p.N + col];
#pragma unroll
                        for (int e = 0; e < 8; ++e) acc[ii][jj][h + e] = old[e] + acc[ii][jj][h + e];
                    }
                }
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int t = tb + 8 * (e >> 2) + (e & 3);
                    if (t < p.M) p.Y[static_cast<int64_t>(t) * p.N + col] = acc[ii][jj][e];
                }
            }
        }
    }
}

template <int EPI>
void launch_ring(bool ring1, const Split3Params & p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(p.m_tiles * p.n_tiles));
    if (ring1) hipLaunchKernelGGL((gemm_split3_kernel<1, EPI>), grid, dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((gemm_split3_kernel<2, EPI>), grid, dim3(kThreads), 0, stream, p);
}

}  // namespace

bool gemm_split3_shape_ok(int32_t N, int32_t K, bool swiglu) {
    return N > 0 && K > 0 && K % kBK == 0 && N % (swiglu ? kBN / 2 : kBN) == 0;
}

int gemm_split3_launch(const uint16_t * W16, int32_t N, int32_t K, const uint16_t * Xs, int32_t M, float * Y,
                       bool accumulate, uint16_t * act, hipStream_t stream) {
    const bool swiglu = act != nullptr;
    if (!W16 || !Xs || M <= 0 || (swiglu ? Y != nullptr || accumulate : Y == nullptr)) {
        return fail(QA_ERR_INVALID, "gemm_split3: invalid arguments");
    }
    if (!gemm_split3_shape_ok(N, K, swiglu)) {
        return fail(QA_ERR_INVALID, "gemm_split3: needs K % 64 == 0 and N % 256 == 0 (SwiGLU: N % 128 == 0)");
    }
    Split3Params p{};
    p.W = W16;
    p.Xs = Xs;
    p.Y = Y;
    p.act = act;
    p.M = M;
    p.N = N;
    p.K = K;
    p.m_tiles = (M + kBM - 1) / kBM;
    p.n_tiles = N / (swiglu ? kBN / 2 : kBN);
    if (static_cast<int64_t>(p.m_tiles) * p.n_tiles > 0x7fffffff) return fail(QA_ERR_INVALID, "gemm_split3: grid too large");
    // two workgroups per CU alternate once the grid holds about two per CU (measured at T = 3913); the
    // accumulating epilogue needs more than the 128 registers per lane that two workgroups per CU allow
    const bool ring1 = static_cast<int64_t>(p.m_tiles) * p.n_tiles >= 384 && !accumulate;
    if (swiglu) launch_ring<kS3Swiglu>(ring1, p, stream);
    else if (accumulate) launch_ring<kS3Accumulate>(ring1, p, stream);
    else launch_ring<kS3Store>(ring1, p, stream);
    QA_LAUNCH_CHECK("gemm_split3_kernel");
    return QA_OK;
}

}  // namespace qa

extern "C" int qa_gemm_split3_bf16(const uint16_t * W_bf16, int32_t out_dim, int32_t in_dim, const uint16_t * x_split,
                                   int32_t rows, float * y, int32_t accumulate, uint16_t * act_split, void * stream) {
    return qa::gemm_split3_launch(W_bf16, out_dim, in_dim, x_split, rows, y, accumulate != 0, act_split,
                                  qa::as_stream(stream));
}
