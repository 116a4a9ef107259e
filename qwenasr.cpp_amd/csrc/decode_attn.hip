// Split-K GQA decode attention over the KV cache (flash-decoding), gfx950.
//
// Replaces the decode half of backend_text_layer_forward_cached_ggml (text-decoder.cpp:435-463):
//   scores = mul_mat(K[0,L), q); soft_max_ext(scores, mask, 1/sqrt(d)); out = mul_mat(cont(V^T), p)
// including the transposed copy of V that the reference materialises on every call (459): V is read
// row-wise here, so each K and V byte of the attended prefix is read from HBM exactly once.
//
// Arithmetic = the reference's GGML graph for the cache dtype (f32 precision):
//   s_j = f32dot(q, K_j) * scale, q rounded to f16 first when K is f16 (GGML's mul_mat converts src1
//   to the f16 dot type of src0); max over j; sum of expf(s_j - max) in double;
//   p_j = expf(s_j - max) * (float)(1 / sum), rounded to f16 when V is f16 (same conversion rule);
//   o = f32 sum of p_j V_j.
// The f16 rounding of the NORMALISED p needs the global max and sum before any PV, so the work is two
// launches over the same (chunk, KV head, stream) grid:
//   scores kernel  K rows of the chunk -> scores of both query heads of the GQA group (workspace) and
//                  the chunk's max m_c and double sum_j expf(s_j - m_c);
//   values kernel  global max M and sum S = sum_c sum_c * exp(m_c - M) from the chunk statistics,
//                  p_j, the chunk's partial o, and the merge: the last workgroup of each
//                  (stream, KV head) adds the partials in a fixed order.
// The two kernels chunk the positions independently: the scores kernel finely (no merge, so many
// workgroups in flight), the values kernel coarsely (its chunks are the merge participants).
// Dropping the p rounding would allow a single-pass launch, but it moves logits by up to ~1e-3 and
// flips greedy near-ties against the reference semantics; identical greedy ids are the contract.
//
// Work decomposition.  One workgroup (4 waves) owns CHUNK consecutive positions of one KV head of one
// stream and serves both query heads of the group (Q head h reads KV head h / 2,
// text-decoder.cpp:725, 1035), so every K/V byte loaded feeds two dot products from registers.
// 16 lanes cover one 128-wide row (8 elements per lane, one 16-byte load for f16); one wave load
// instruction fetches 4 consecutive rows (1 KB of f16).  A workgroup issues every load of its chunk
// before the first arithmetic, so the whole chunk is in flight at once.
// blockIdx.x = chunk * n_kv + kv_head: consecutive workgroups (round-robin over the 8 XCDs) walk the
// KV heads of one chunk.
//
// Merge without fences.  The partial o of a chunk is published with agent-scope atomic stores and
// read back by the merging workgroup with agent-scope atomic loads (both coherent across XCDs by
// themselves), ordered by a vmcnt wait before the counter increment.  A release/acquire fence would
// order plain stores instead, at the price of writing back and invalidating the whole L2 of the XCD
// in every workgroup, which costs more than the attention itself.  The counter is reset by the
// merging workgroup, so the workspace never needs clearing between calls.
//
// Fused mode (the decode step of the runtime): the scores kernel takes the raw q|k|v projection row
// and does the append itself.  Every workgroup normalises and rotates its two query heads (the same
// function, hence the same bits, as the append kernel); the workgroup that owns the new position
// normalises and rotates k, casts k and v to the cache dtype and writes both rows into the cache, and
// uses the new K row from LDS.  The values kernel then reads the new V row from the cache: the
// reference's append-then-attend order (the cpy nodes precede attention, text-decoder.cpp:432-433)
// without a separate append launch.
#include "decode_attn_body.hpp"
#include "ops.hpp"
#include "prep.hpp"

#include <cmath>
#include <cstdlib>
#include <mutex>

namespace qa {
namespace {

// One pass per launch (the bodies are in decode_attn_body.hpp, shared with the persistent decode step).
template <typename CT, bool R16, int CHUNK, bool FUSED>
__global__ __launch_bounds__(kThreads) void decode_scores_kernel(DecodeParams p, RopeTable rope) {
    decode_scores_body<CT, R16, CHUNK, FUSED, false>(p, rope, blockIdx.x, blockIdx.y);
}

template <typename CT, bool R16, int CHUNK, int SR, int MB>
__global__ __launch_bounds__(kThreads) void decode_values_kernel(DecodeParams p) {
    decode_values_body<CT, R16, CHUNK, SR, MB, false>(p, blockIdx.x, blockIdx.y);
}

template <typename CT, bool R16, bool FUSED>
void launch_scores(int chunk, dim3 grid, const DecodeParams & p, const RopeTable & rope, hipStream_t stream) {
    switch (chunk) {
        case 32: hipLaunchKernelGGL((decode_scores_kernel<CT, R16, 32, FUSED>), grid, dim3(kThreads), 0, stream, p, rope); break;
        case 64: hipLaunchKernelGGL((decode_scores_kernel<CT, R16, 64, FUSED>), grid, dim3(kThreads), 0, stream, p, rope); break;
        case 144: hipLaunchKernelGGL((decode_scores_kernel<CT, R16, 144, FUSED>), grid, dim3(kThreads), 0, stream, p, rope); break;
        case 160: hipLaunchKernelGGL((decode_scores_kernel<CT, R16, 160, FUSED>), grid, dim3(kThreads), 0, stream, p, rope); break;
        case 192: hipLaunchKernelGGL((decode_scores_kernel<CT, R16, 192, FUSED>), grid, dim3(kThreads), 0, stream, p, rope); break;
        case 256: hipLaunchKernelGGL((decode_scores_kernel<CT, R16, 256, FUSED>), grid, dim3(kThreads), 0, stream, p, rope); break;
        default: hipLaunchKernelGGL((decode_scores_kernel<CT, R16, 128, FUSED>), grid, dim3(kThreads), 0, stream, p, rope); break;
    }
}

template <typename CT, bool R16, int CHUNK, int MB>
void launch_values_sr(int sr, dim3 grid, const DecodeParams & p, hipStream_t stream) {
    switch (sr) {
        case 1: hipLaunchKernelGGL((decode_values_kernel<CT, R16, CHUNK, 1, MB>), grid, dim3(kThreads), 0, stream, p); break;
        case 2: hipLaunchKernelGGL((decode_values_kernel<CT, R16, CHUNK, 2, MB>), grid, dim3(kThreads), 0, stream, p); break;
        case 4: hipLaunchKernelGGL((decode_values_kernel<CT, R16, CHUNK, 4, MB>), grid, dim3(kThreads), 0, stream, p); break;
        default: hipLaunchKernelGGL((decode_values_kernel<CT, R16, CHUNK, 8, MB>), grid, dim3(kThreads), 0, stream, p); break;
    }
}

template <typename CT, bool R16, int CHUNK>
void launch_values_mb(int sr, int mb, dim3 grid, const DecodeParams & p, hipStream_t stream) {
    if (mb <= 8) launch_values_sr<CT, R16, CHUNK, 8>(sr, grid, p, stream);
    else if (mb <= 16) launch_values_sr<CT, R16, CHUNK, 16>(sr, grid, p, stream);
    else launch_values_sr<CT, R16, CHUNK, 40>(sr, grid, p, stream);
}

// false (nothing launched) for a chunk the values kernel is not instantiated for
template <typename CT, bool R16>
bool launch_values(int chunk, int sr, int mb, dim3 grid, const DecodeParams & p, hipStream_t stream) {
    switch (chunk) {
        case 32: launch_values_mb<CT, R16, 32>(sr, mb, grid, p, stream); return true;
        case 64: launch_values_mb<CT, R16, 64>(sr, mb, grid, p, stream); return true;
        case 128: launch_values_mb<CT, R16, 128>(sr, mb, grid, p, stream); return true;
        case 256: launch_values_mb<CT, R16, 256>(sr, mb, grid, p, stream); return true;
        default: return false;
    }
}

template <typename CT, bool R16>
bool launch_both(const Chunks & ch, bool fused, int32_t n_kv, int32_t n_streams, DecodeParams p, const RopeTable & rope,
                 hipStream_t stream) {
    p.stat_chunk = ch.scores;
    const dim3 gs(static_cast<unsigned>((p.max_len + ch.scores - 1) / ch.scores * n_kv), static_cast<unsigned>(n_streams));
    const dim3 gv(static_cast<unsigned>((p.max_len + ch.values - 1) / ch.values * n_kv), static_cast<unsigned>(n_streams));
    if (fused) launch_scores<CT, R16, true>(ch.scores, gs, p, rope, stream);
    else launch_scores<CT, R16, false>(ch.scores, gs, p, rope, stream);
    return launch_values<CT, R16>(ch.values, values_stat_regs(p.max_seq, ch.scores),
                                  values_merge_loads(p.max_seq, ch.values), gv, p, stream);
}

int launch_decode(DecodeParams p, bool fused, const RopeTable & rope, const qa_kv_layout & layout,
                  int32_t n_streams, void * workspace, size_t workspace_bytes, hipStream_t stream) {
    const Chunks ch = pick_chunks(layout);
    if (ch.values != 32 && ch.values != 64 && ch.values != 128 && ch.values != 256) {
        return fail(QA_ERR_INVALID, "decode attention: no values kernel for the chosen chunk");
    }
    if (!set_workspace(p, layout, workspace, workspace_bytes)) {
        return fail(QA_ERR_INVALID, "decode attention: workspace too small for the cache capacity");
    }
    const bool ok = layout.cache_type == QA_CACHE_F16
                        ? launch_both<_Float16, true>(ch, fused, layout.n_kv_heads, n_streams, p, rope, stream)
                        : launch_both<float, false>(ch, fused, layout.n_kv_heads, n_streams, p, rope, stream);
    if (!ok) return fail(QA_ERR_INVALID, "decode attention: no values kernel for the chosen chunk");
    QA_LAUNCH_CHECK("decode attention kernels");
    return QA_OK;
}

int check_shape(const qa_kv_layout & layout, int32_t n_streams, int32_t max_len, int32_t n_heads, int32_t layer) {
    if (layout.head_dim != kHeadDim || n_heads != kRep * layout.n_kv_heads) {
        return fail(QA_ERR_INVALID, "decode attention: only head_dim 128 with 2 query heads per KV head");
    }
    if (n_streams <= 0 || n_streams > layout.n_streams || max_len <= 0 || max_len > layout.max_seq ||
        layer < 0 || layer >= layout.n_layers) {
        return fail(QA_ERR_INVALID, "decode attention: invalid streams, length or layer");
    }
    return QA_OK;
}

}  // namespace

int decode_attn_launch(const float * q, int32_t q_stride, const void * cache, const qa_kv_layout & layout,
                       int32_t layer, const int32_t * lens, int32_t lens_add, int32_t n_streams,
                       int32_t max_len, int32_t n_heads, float scale, float * out, void * workspace,
                       size_t workspace_bytes, hipStream_t stream) {
    const int rc = check_shape(layout, n_streams, max_len, n_heads, layer);
    if (rc != QA_OK) return rc;
    DecodeParams p{};
    p.q = q;
    p.cache = const_cast<void *>(cache);
    p.out = out;
    p.lens = lens;
    p.lens_add = lens_add;
    p.q_stride = q_stride;
    p.out_stride = n_heads * kHeadDim;
    p.n_heads = n_heads;
    p.layer = layer;
    p.max_len = max_len;
    p.scale = scale;
    return launch_decode(p, false, RopeTable{}, layout, n_streams, workspace, workspace_bytes, stream);
}

int decode_step_attn_launch(const float * qkv, const float * q_norm_w, const float * k_norm_w, void * cache,
                            const qa_kv_layout & layout, int32_t layer, const int32_t * n_past, int32_t n_streams,
                            int32_t max_len, int32_t n_heads, float rope_theta, float eps, float scale, float * out,
                            void * workspace, size_t workspace_bytes, hipStream_t stream) {
    const int rc = check_shape(layout, n_streams, max_len, n_heads, layer);
    if (rc != QA_OK) return rc;
    DecodeParams p{};
    p.q = qkv;
    p.cache = cache;
    p.out = out;
    p.lens = n_past;
    p.lens_add = 1;
    p.q_norm_w = q_norm_w;
    p.k_norm_w = k_norm_w;
    p.eps = eps;
    p.q_stride = (n_heads + 2 * layout.n_kv_heads) * kHeadDim;
    p.out_stride = n_heads * kHeadDim;
    p.n_heads = n_heads;
    p.layer = layer;
    p.max_len = max_len;
    p.scale = scale;
    return launch_decode(p, true, make_rope_table(rope_theta), layout, n_streams, workspace, workspace_bytes, stream);
}

// ---- allocation-free variant (qa_decode_step_attn_noalloc)
// The workspace of the decode step lives in this file-scope device array instead of memory the caller
// or the library allocates.  Each GPU holds its own copy, at its own address, until the process ends.
// Host code never passes `scratch` itself to a kernel (on the host that name is a stand-in, not a
// device address): the address comes from hipGetSymbolAddress, once per device, with the device
// current, and is kept in noalloc_ptrs.
namespace {

constexpr size_t kNoAllocScratchBytes = QA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
void * noalloc_ptrs[kMaxDevices] = {};
std::mutex noalloc_mutex;

// The address is resolved on the device's first call, or earlier by qa_decode_noalloc_prepare (the
// decoder calls it at creation).  A first call made while `stream` is being captured is refused, so the
// lookup never runs inside a capture: callers that capture make one eager call (or the prepare call) first.
int noalloc_scratch(void ** out, hipStream_t stream) {
    int device = 0;
    QA_HIP(hipGetDevice(&device));
    if (device < 0 || device >= kMaxDevices) return fail(QA_ERR_DEVICE, "decode attention: device index out of range");
    std::lock_guard<std::mutex> lock(noalloc_mutex);
    if (!noalloc_ptrs[device] && stream) {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        QA_HIP(hipStreamIsCapturing(stream, &st));
        if (st != hipStreamCaptureStatusNone) {
            return fail(QA_ERR_INVALID, "qa_decode_step_attn_noalloc: the scratch address of this device is not "
                                        "resolved yet; call qa_decode_noalloc_prepare (or the entry point once) "
                                        "outside stream capture first");
        }
    }
    if (!noalloc_ptrs[device]) {
        void * p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e, "hipGetSymbolAddress (decode attention scratch)");
        noalloc_ptrs[device] = p;
    }
    *out = noalloc_ptrs[device];
    return QA_OK;
}

// Zeroes n 32-bit words with vector stores (a kernel rather than hipMemsetAsync, so a captured call
// holds no memset node).
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t * p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) p[i] = 0u;
}

}  // namespace

size_t decode_attn_workspace(int32_t n_streams, int32_t n_kv_heads, int32_t max_seq) {
    if (n_streams <= 0 || n_kv_heads <= 0 || max_seq <= 0) return 0;
    return workspace_layout(n_streams, n_kv_heads, max_seq).total;
}

}  // namespace qa

extern "C" size_t qa_decode_attn_workspace_bytes(int32_t n_streams, int32_t n_heads, int32_t max_seq) {
    if (n_heads <= 0 || n_heads % qa::kRep != 0) return 0;
    return qa::decode_attn_workspace(n_streams, n_heads / qa::kRep, max_seq);
}

extern "C" int qa_decode_attn(const float * q, const void * cache, const qa_kv_layout * layout, int32_t layer,
                              const int32_t * lens, int32_t n_streams, int32_t max_len, int32_t n_heads,
                              float scale, float * out, void * workspace, size_t workspace_bytes, void * stream) {
    using namespace qa;
    if (qa_kv_layout_check(layout) != QA_OK) return QA_ERR_INVALID;
    if (!q || !cache || !lens || !out) return fail(QA_ERR_INVALID, "qa_decode_attn: null pointer");
    return decode_attn_launch(q, n_heads * kHeadDim, cache, *layout, layer, lens, 0, n_streams, max_len,
                              n_heads, scale, out, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int qa_decode_step_attn(const float * qkv, const float * q_norm_w, const float * k_norm_w, void * cache,
                                   const qa_kv_layout * layout, int32_t layer, const int32_t * n_past,
                                   int32_t n_streams, int32_t max_len, int32_t n_heads, float rope_theta, float eps,
                                   float scale, float * out, void * workspace, size_t workspace_bytes, void * stream) {
    using namespace qa;
    if (qa_kv_layout_check(layout) != QA_OK) return QA_ERR_INVALID;
    if (!qkv || !q_norm_w || !k_norm_w || !cache || !n_past || !out) {
        return fail(QA_ERR_INVALID, "qa_decode_step_attn: null pointer");
    }
    return decode_step_attn_launch(qkv, q_norm_w, k_norm_w, cache, *layout, layer, n_past, n_streams, max_len, n_heads,
                                   rope_theta, eps, scale, out, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int qa_decode_noalloc_prepare(void) {
    void * base = nullptr;
    return qa::noalloc_scratch(&base, nullptr);
}

extern "C" int qa_decode_step_attn_noalloc(const float * qkv, const float * q_norm_w, const float * k_norm_w,
                                           void * cache, const qa_kv_layout * layout, int32_t layer,
                                           const int32_t * n_past, int32_t n_streams, int32_t max_len, int32_t n_heads,
                                           float rope_theta, float eps, float scale, float * out, void * stream) {
    using namespace qa;
    if (qa_kv_layout_check(layout) != QA_OK) return QA_ERR_INVALID;
    if (!qkv || !q_norm_w || !k_norm_w || !cache || !n_past || !out) {
        return fail(QA_ERR_INVALID, "qa_decode_step_attn_noalloc: null pointer");
    }
    if (n_heads <= 0 || n_heads % kRep != 0) return fail(QA_ERR_INVALID, "qa_decode_step_attn_noalloc: invalid n_heads");
    const Workspace w = workspace_layout(layout->n_streams, layout->n_kv_heads, layout->max_seq);
    if (w.total > kNoAllocScratchBytes) {
        return fail(QA_ERR_INVALID, "qa_decode_step_attn_noalloc: the cache capacity needs " + std::to_string(w.total) +
                                        " bytes of scratch, more than its maximum of " +
                                        std::to_string(kNoAllocScratchBytes));
    }
    int rc = check_shape(*layout, n_streams, max_len, n_heads, layer);
    if (rc != QA_OK) return rc;
    void * base = nullptr;
    rc = noalloc_scratch(&base, as_stream(stream));
    if (rc != QA_OK) return rc;
    // A previous call may have used another capacity, whose partials now lie where this layout keeps
    // its merge counters: clear this layout's counters on every call.
    const int64_t n_words = static_cast<int64_t>((w.total - w.counters) / sizeof(uint32_t));
    hipLaunchKernelGGL(zero_words_kernel, dim3(static_cast<unsigned>((n_words + 255) / 256)), dim3(256), 0,
                       as_stream(stream), reinterpret_cast<uint32_t *>(static_cast<char *>(base) + w.counters), n_words);
    QA_LAUNCH_CHECK("zero_words_kernel");
    return decode_step_attn_launch(qkv, q_norm_w, k_norm_w, cache, *layout, layer, n_past, n_streams, max_len, n_heads,
                                   rope_theta, eps, scale, out, base, w.total, as_stream(stream));
}
