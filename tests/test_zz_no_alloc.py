"""qa_decode_step_attn_noalloc (workspace in the library's file-scope device scratch) against
qa_decode_step_attn (caller's workspace): two calls in a row, the second with a smaller cache capacity
and fewer streams, so its merge counters sit where the first call's partial outputs were.  Same kernels,
so the outputs and the whole cache must be bit-identical; the output is also held to the attention
tolerance of the oracle.  Layouts whose workspace exceeds the scratch are rejected before any launch."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SCALE = 1.0 / np.sqrt(128.0)


@pytest.fixture(scope="module", autouse=True)
def _gpu(qa):
    assert qa.device_count() > 0, "no HIP device: GPU tests need the MI355X"


def step_pair(qa, orc, n_past, max_seq, f16, seed):
    """One decode step of layer 1 through both entry points on identical caches."""
    S = len(n_past)
    lay = qa.KvLayout(2, S, 8, 128, max_seq, qa.QA_CACHE_F16 if f16 else qa.QA_CACHE_F32)
    rng = np.random.default_rng(seed)
    qkv = (rng.standard_normal((S, 4096)) * 0.7).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    dt = np.float16 if f16 else np.float32
    host = np.zeros((2, 2, S, 8, max_seq, 128), dt)
    for s, P in enumerate(n_past):
        host[1, :, s, :, :P] = rng.standard_normal((2, 8, P, 128))
    d_qkv, d_qn, d_kn = (qa.DeviceArray.from_numpy(a) for a in (qkv, qn, kn))
    d_np = qa.DeviceArray.from_numpy(np.array(n_past, np.int32))
    results = []
    for noalloc in (False, True):
        cache = qa.DeviceArray.from_numpy(host)
        out = qa.DeviceArray((S, 2048), np.float32)
        args = (d_qkv.ptr, d_qn.ptr, d_kn.ptr, cache.ptr, C.byref(lay), 1, d_np.ptr, S, max(n_past) + 1, 16, 1.0e6,
                1e-6, SCALE, out.ptr)
        print(f"decode step noalloc={noalloc} f16={f16} streams={S} max_seq={max_seq}", flush=True)
        if noalloc:
            qa.check(qa.lib.qa_decode_step_attn_noalloc(*args, None))
        else:
            ws_bytes = qa.lib.qa_decode_attn_workspace_bytes(S, 16, max_seq)
            ws = qa.DeviceArray(ws_bytes, np.uint8)
            qa.check(qa.lib.qa_decode_step_attn(*args, ws.ptr, ws_bytes, None))
        qa.synchronize()
        results.append((cache.numpy(), out.numpy().reshape(S, 16, 128)))
    (c0, o0), (c1, o1) = results
    np.testing.assert_array_equal(c0.view(np.uint16 if f16 else np.uint32), c1.view(np.uint16 if f16 else np.uint32))
    np.testing.assert_array_equal(o0.view(np.uint32), o1.view(np.uint32))
    for s, P in enumerate(n_past):
        q, _ = orc.qk_prep(qkv[s:s + 1, :2048].reshape(1, 16, 128), qkv[s:s + 1, 2048:3072].reshape(1, 8, 128),
                           qn, kn, P, 1.0e6, 1e-6)
        k = c1[1, 0, s, :, :P + 1].astype(np.float32)
        v = c1[1, 1, s, :, :P + 1].astype(np.float32)
        ref = orc.cache_attention(k, v, q, P, f16)[0]
        err = float(np.abs(o1[s] - ref).max())
        rel = float(np.linalg.norm(o1[s] - ref) / np.linalg.norm(ref))
        assert err <= 2e-3 and rel <= 1e-3, (s, err, rel)


def test_noalloc_matches_workspace_entry_point_over_two_calls(qa, orc):
    step_pair(qa, orc, [1200, 37, 3000, 640, 2047], 3100, True, 1)     # 5 streams, capacity 3100
    step_pair(qa, orc, [250], 300, True, 2)                            # then 1 stream, capacity 300
    step_pair(qa, orc, [90, 5], 120, False, 3)                         # and an f32 cache


def test_noalloc_matches_at_long_single_stream_capacities(qa, orc):
    # one stream at capacities 4600 and 6000: the scores kernel then takes 144- and 192-position chunks
    step_pair(qa, orc, [4499], 4600, True, 4)
    step_pair(qa, orc, [5900], 6000, True, 5)


def test_noalloc_rejects_capacity_beyond_scratch(qa):
    lay = qa.KvLayout(1, 32, 8, 128, 8192, qa.QA_CACHE_F16)
    need = qa.lib.qa_decode_attn_workspace_bytes(32, 16, 8192)
    assert need > qa.QA_NOALLOC_SCRATCH_BYTES
    small = qa.DeviceArray(4096, np.float32)     # real buffers; the call is rejected before any launch
    p = small.ptr
    rc = qa.lib.qa_decode_step_attn_noalloc(p, p, p, p, C.byref(lay), 0, p, 1, 16, 16, 1.0e6, 1e-6, SCALE, p, None)
    assert rc == qa.QA_ERR_INVALID and b"maximum" in qa.lib.qa_last_error()
    fits = qa.lib.qa_decode_attn_workspace_bytes(32, 16, 4000)        # config 4's capacity fits
    assert fits <= qa.QA_NOALLOC_SCRATCH_BYTES


def test_noalloc_prepare_is_idempotent(qa):
    """The set-up call resolves the scratch address of the current device; later calls (and the decoder's
    own call at creation) find it resolved."""
    assert qa.lib.qa_decode_noalloc_prepare() == qa.QA_OK
    assert qa.lib.qa_decode_noalloc_prepare() == qa.QA_OK
