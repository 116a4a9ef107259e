// Host side of the persistent decode step (the kernel and its design: decode_persist.hpp): the plan (which
// unit holds the decoder's kernel, the resident grid) and the launch.
#include "decode_persist.hpp"

#include <algorithm>
#include <string>

namespace qa {
namespace {

struct Unit {
    int (*find)(const PersistPlanIn &, int *);
    int (*launch)(const PersistLaunch &, hipStream_t);
};

#define QA_PERSIST_ENTRY(NAME) Unit{persist_find_##NAME, persist_launch_##NAME},
const Unit kUnits[] = {QA_PERSIST_UNITS(QA_PERSIST_ENTRY)};

}  // namespace

size_t persist_ws_stride(const qa_kv_layout & layout) {
    return align256(workspace_layout(layout.n_streams, layout.n_kv_heads, layout.max_seq).total);
}

size_t persist_sync_bytes(int32_t grid) {
    return sizeof(uint32_t) * static_cast<size_t>(SyncLayout{(grid + kGroup - 1) / kGroup}.words());
}

int persist_error_word_offset(int32_t grid) {
    return SyncLayout{(grid + kGroup - 1) / kGroup}.error();
}

int persist_plan(const PersistPlanIn & in, int32_t * grid) {
    if (in.layout.n_streams != 1) return fail(QA_ERR_INVALID, "persistent decode step: single-stream decoders only");
    int per_cu = 0, rc = QA_ERR_INVALID;
    for (const Unit & u : kUnits) {
        rc = u.find(in, &per_cu);
        if (rc != QA_ERR_INVALID) break;
    }
    if (rc == QA_ERR_INVALID) {
        const Chunks ch = pick_chunks(in.layout);
        return fail(QA_ERR_INVALID, "persistent decode step: no kernel for this model shape (hidden " +
                                        std::to_string(in.hidden) + ", q_dim " + std::to_string(in.q_dim) +
                                        ", intermediate " + std::to_string(in.inter) + ") and tiling (scores chunk " +
                                        std::to_string(ch.scores) + ", values chunk " + std::to_string(ch.values) + ")");
    }
    if (rc != QA_OK) return rc;
    if (per_cu < 1) return fail(QA_ERR_DEVICE, "persistent decode step: the kernel does not fit on a CU");
    int device = 0, cus = 0;
    QA_HIP(hipGetDevice(&device));
    QA_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
    *grid = cus;   // one workgroup per CU (the kernel is built for one wave per SIMD)
    return QA_OK;
}

int persist_layers_launch(const PersistLaunch & a, hipStream_t stream) {
    for (const Unit & u : kUnits) {
        const int rc = u.launch(a, stream);
        if (rc != QA_ERR_INVALID) return rc;
    }
    return fail(QA_ERR_INVALID, "persistent decode step: no kernel for this configuration");
}

}  // namespace qa
