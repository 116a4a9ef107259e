"""Kernel-level parity of the HIP path against the CPU oracle, through the C ABI.

Device memory is allocated and copied through the library's own C ABI (qa_device_malloc and
friends), so these tests load exactly one HIP runtime: the one libqwenasr_amd.so links.  Every
computation is a qa_* entry point.  Bars: cache slots, positions and lengths
bit-exact; attention within 2e-3 max-abs and 1e-3 relative-L2 with f32 accumulation.  The append
kernel is held to bit-exactness of the whole cache (written rows and untouched rows alike).
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ATOL, RTOL_L2 = 2e-3, 1e-3
SCALE = 1.0 / np.sqrt(128.0)
NULL_STREAM = None


def check_close(got, ref, atol=ATOL, rtol_l2=RTOL_L2):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref).max()
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert err <= atol and rel <= rtol_l2, (err, rel)
    return err, rel


@pytest.fixture(scope="module", autouse=True)
def _gpu(qa):
    assert qa.device_count() > 0, "no HIP device: GPU tests need the MI355X"
    arch = C.create_string_buffer(64)
    qa.check(qa.lib.qa_device_arch(arch, 64))
    print("device:", arch.value.decode(), flush=True)


def dev(qa, a):
    return qa.DeviceArray.from_numpy(a)


def zeros(qa, shape, dtype=np.float32):
    return qa.DeviceArray(shape, dtype)


def layout(qa, n_layers, n_streams, max_seq, f16):
    return qa.KvLayout(n_layers, n_streams, 8, 128, max_seq, qa.QA_CACHE_F16 if f16 else qa.QA_CACHE_F32)


class Cache:
    """Host mirror [layer][kv][stream][head][pos][dim] of one device K+V allocation."""

    def __init__(self, qa, lay):
        self.lay = lay
        dt = np.float16 if lay.cache_type == qa.QA_CACHE_F16 else np.float32
        self.host = np.zeros((lay.n_layers, 2, lay.n_streams, lay.n_kv_heads, lay.max_seq, lay.head_dim), dt)
        assert self.host.nbytes == qa.lib.qa_kv_cache_bytes(C.byref(lay))
        self.dev = qa.DeviceArray(self.host.shape, dt)

    def fill(self, rng, layer, stream_lens):
        """Random K/V rows [0, L) per stream at `layer`; returns the f32 values actually stored."""
        vals = {}
        for s, L in enumerate(stream_lens):
            k = rng.standard_normal((8, L, 128)).astype(np.float32)
            v = rng.standard_normal((8, L, 128)).astype(np.float32)
            self.host[layer, 0, s, :, :L] = k
            self.host[layer, 1, s, :, :L] = v
            vals[s] = (self.host[layer, 0, s, :, :L].astype(np.float32), self.host[layer, 1, s, :, :L].astype(np.float32))
        self.dev.upload(self.host)
        return vals

    def read(self):
        return self.dev.numpy().astype(np.float32)

    @property
    def ptr(self):
        return self.dev.ptr


# ------------------------------------------------------------------------------------------ append
@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("T,n_past", [(1, [0, 17, 4167]), (5, [3, 100, 4000]), (156, [0])])
def test_kv_append_bit_exact(qa, orc, f16, T, n_past):
    S = len(n_past)
    lay = layout(qa, 2, S, 4169, f16)
    cache = Cache(qa, lay)
    rng = np.random.default_rng(T * 7 + S)
    qkv = (rng.standard_normal((S * T, 4096)) * 0.7).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    d_qkv, d_qn, d_kn = dev(qa, qkv), dev(qa, qn), dev(qa, kn)
    d_q = zeros(qa, (S * T, 2048))
    d_np = dev(qa, np.array(n_past, np.int32))
    print(f"append f16={f16} T={T} n_past={n_past}", flush=True)
    qa.check(qa.lib.qa_kv_append(d_qkv.ptr, d_qn.ptr, d_kn.ptr, d_q.ptr, cache.ptr, C.byref(lay), 1, d_np.ptr, S, T,
                                 16, 1.0e6, 1e-6, NULL_STREAM))
    qa.synchronize()
    got = cache.read()
    q_got = d_q.numpy()
    expect = np.zeros_like(got)
    for s in range(S):
        rows = qkv[s * T:(s + 1) * T]
        q, k = orc.qk_prep(rows[:, :2048].reshape(T, 16, 128), rows[:, 2048:3072].reshape(T, 8, 128), qn, kn,
                           n_past[s], 1.0e6, 1e-6)
        v = rows[:, 3072:].reshape(T, 8, 128)
        if f16:
            k = k.astype(np.float16).astype(np.float32)   # numpy's cast is RNE, pinned against the oracle's
            v = v.astype(np.float16).astype(np.float32)
        expect[1, 0, s, :, n_past[s]:n_past[s] + T] = k.transpose(1, 0, 2)
        expect[1, 1, s, :, n_past[s]:n_past[s] + T] = v.transpose(1, 0, 2)
        np.testing.assert_array_equal(q_got[s * T:(s + 1) * T].view(np.uint32), q.reshape(T, 2048).view(np.uint32))
    np.testing.assert_array_equal(got.view(np.uint32), expect.view(np.uint32))


# ------------------------------------------------------------------------------------------ decode
def _decode(qa, q_dev, cache, lay, layer, lens, max_len, out, ws, ws_bytes):
    d_lens = dev(qa, np.array(lens, np.int32))
    qa.check(qa.lib.qa_decode_attn(q_dev.ptr, cache.ptr, C.byref(lay), layer, d_lens.ptr, len(lens), max_len, 16, SCALE,
                                   out.ptr, ws.ptr, ws_bytes, NULL_STREAM))
    qa.synchronize()
    return out.numpy().reshape(len(lens), 16, 128)


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("lens", [[1], [2], [63], [64], [65], [157], [1000], [4096], [4186], [4500], [5000], [6000],
                                  [8000], [156, 3913, 700, 1, 2048]])
def test_decode_attention(qa, orc, f16, lens):
    S = len(lens)
    max_len = max(lens)
    lay = layout(qa, 3, S, max_len + 3, f16)
    cache = Cache(qa, lay)
    rng = np.random.default_rng(sum(lens))
    vals = cache.fill(rng, 2, lens)
    q = rng.standard_normal((S, 16, 128)).astype(np.float32)
    d_q, d_out = dev(qa, q), zeros(qa, (S, 2048))
    ws_bytes = qa.lib.qa_decode_attn_workspace_bytes(S, 16, lay.max_seq)
    ws = zeros(qa, ws_bytes, np.uint8)
    print(f"decode f16={f16} lens={lens}", flush=True)
    for rep in range(2):   # the second call checks the counters were left at zero
        got = _decode(qa, d_q, cache, lay, 2, lens, max_len, d_out, ws, ws_bytes)
        for s, L in enumerate(lens):
            k, v = vals[s]
            ref = orc.cache_attention(k, v, q[s:s + 1], L - 1, f16)[0]
            check_close(got[s], ref)


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("S", [1, 2])
def test_decode_attention_growing_lengths_one_workspace(qa, orc, f16, S):
    """One workspace, never cleared between calls, while the prefix grows across chunk boundaries
    (1 -> many chunks, and 32/64/128/144-row boundaries; one stream at this capacity takes 144-row
    scores chunks, two take 128): every call must match the oracle, so the merge counters stay where
    the capacity put them and are left at zero by each call."""
    cap = 4200
    lay = layout(qa, 1, S, cap, f16)
    cache = Cache(qa, lay)
    rng = np.random.default_rng(7)
    vals = cache.fill(rng, 0, [cap] * S)
    q = rng.standard_normal((S, 16, 128)).astype(np.float32)
    d_q, d_out = dev(qa, q), zeros(qa, (S, 2048))
    ws_bytes = qa.lib.qa_decode_attn_workspace_bytes(S, 16, cap)
    ws = zeros(qa, ws_bytes, np.uint8)
    for lens2 in ([1, 3], [31, 33], [32, 64], [65, 63], [127, 129], [130, 1], [144, 145], [288, 289], [1023, 2047],
                  [4096, 4100], [4200, 200], [5, 6]):
        lens = lens2[:S]
        print(f"decode growing f16={f16} lens={lens}", flush=True)
        got = _decode(qa, d_q, cache, lay, 0, lens, max(lens), d_out, ws, ws_bytes)
        for s, L in enumerate(lens):
            k, v = vals[s]
            ref = orc.cache_attention(k[:, :L], v[:, :L], q[s:s + 1], L - 1, f16)[0]
            check_close(got[s], ref)


@pytest.mark.parametrize("f16,L", [(True, 9000), (False, 9000), (True, 16385), (True, 40000)])
def test_decode_attention_long_context(qa, orc, f16, L):
    """Long single-stream contexts: the capacity selects the values kernel's register budgets (chunk
    statistics held in 2-8 register slots plus the loop beyond them at 40000, merge rounds of 40 loads
    over 36-157 participants), so every variant is held to the same bar."""
    lay = layout(qa, 1, 1, L + 3, f16)
    cache = Cache(qa, lay)
    rng = np.random.default_rng(L)
    vals = cache.fill(rng, 0, [L])
    q = rng.standard_normal((1, 16, 128)).astype(np.float32)
    d_q, d_out = dev(qa, q), zeros(qa, (1, 2048))
    ws_bytes = qa.lib.qa_decode_attn_workspace_bytes(1, 16, lay.max_seq)
    ws = zeros(qa, ws_bytes, np.uint8)
    print(f"decode long f16={f16} L={L}", flush=True)
    k, v = vals[0]
    ref = orc.cache_attention(k, v, q, L - 1, f16)[0]
    for rep in range(2):
        got = _decode(qa, d_q, cache, lay, 0, [L], L, d_out, ws, ws_bytes)
        check_close(got[0], ref)


_FORCED_CHUNK_CHILD = r"""
import ctypes as C, os, sys
import numpy as np
root = sys.argv[1]
sys.path[:0] = [os.path.join(root, "qwenasr.cpp_amd"), os.path.join(root, "oracle")]
import qwenasr_amd as qa, qa_oracle as orc
scale = 1.0 / np.sqrt(128.0)
worst = 0.0
for f16 in (True, False):
    for lens in ([1000], [4186], [157, 3000]):
        S, L = len(lens), max(lens)
        lay = qa.KvLayout(1, S, 8, 128, L + 3, qa.QA_CACHE_F16 if f16 else qa.QA_CACHE_F32)
        rng = np.random.default_rng(L + S)
        host = np.zeros((1, 2, S, 8, L + 3, 128), np.float16 if f16 else np.float32)
        for s, n in enumerate(lens):
            host[0, :, s, :, :n] = rng.standard_normal((2, 8, n, 128))
        q = rng.standard_normal((S, 16, 128)).astype(np.float32)
        cache, d_q = qa.DeviceArray.from_numpy(host), qa.DeviceArray.from_numpy(q)
        d_lens, out = qa.DeviceArray.from_numpy(np.array(lens, np.int32)), qa.DeviceArray((S, 2048))
        wsb = qa.lib.qa_decode_attn_workspace_bytes(S, 16, lay.max_seq)
        ws = qa.DeviceArray(wsb, np.uint8)
        print(f"forced chunks f16={f16} lens={lens}", flush=True)
        for rep in range(2):
            qa.check(qa.lib.qa_decode_attn(d_q.ptr, cache.ptr, C.byref(lay), 0, d_lens.ptr, S, L, 16, scale, out.ptr,
                                           ws.ptr, wsb, None))
            got = out.numpy().reshape(S, 16, 128)
            for s, n in enumerate(lens):
                k = host[0, 0, s, :, :n].astype(np.float32)
                v = host[0, 1, s, :, :n].astype(np.float32)
                ref = orc.cache_attention(k, v, q[s:s + 1], n - 1, f16)[0]
                err = float(np.abs(got[s] - ref).max())
                rel = float(np.linalg.norm(got[s] - ref) / np.linalg.norm(ref))
                assert err <= 2e-3 and rel <= 1e-3, (f16, lens, s, err, rel)
                worst = max(worst, err)
print(f"forced chunks ok, max abs err {worst:.2e}", flush=True)
"""


@pytest.mark.parametrize("chunk,vchunk", [("256", "0"), ("144", "144"), ("32", "256")])
def test_decode_attention_forced_chunks(qa, chunk, vchunk):
    """The tuning overrides QA_DECODE_CHUNK / QA_DECODE_VCHUNK (read once per process, so each case runs
    in a child process): a forced 256-position scores chunk, and a values override the values kernel has
    no instantiation for (144: ignored, the capacity's choice stays), both held to the oracle."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, QA_DECODE_CHUNK=chunk, QA_DECODE_VCHUNK=vchunk)
    r = subprocess.run([sys.executable, "-c", _FORCED_CHUNK_CHILD, root], env=env, capture_output=True, text=True,
                       timeout=110)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "forced chunks ok" in r.stdout


def test_decode_attention_rejects_small_workspace(qa):
    lay = layout(qa, 1, 1, 4096, True)
    cache = Cache(qa, lay)
    d_q, d_out = zeros(qa, (1, 2048)), zeros(qa, (1, 2048))
    d_lens = dev(qa, np.array([100], np.int32))
    small = qa.lib.qa_decode_attn_workspace_bytes(1, 16, 1000)
    ws = zeros(qa, small, np.uint8)
    rc = qa.lib.qa_decode_attn(d_q.ptr, cache.ptr, C.byref(lay), 0, d_lens.ptr, 1, 100, 16, 0.1, d_out.ptr, ws.ptr,
                               small, NULL_STREAM)
    assert rc == qa.QA_ERR_INVALID and b"workspace" in qa.lib.qa_last_error()


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("n_past", [[0], [31], [63], [64], [156], [4095], [4185], [6100], [156, 3912, 700, 0, 2047, 31]])
def test_decode_step_fused_equals_append_then_attend(qa, orc, f16, n_past):
    """qa_decode_step_attn == qa_kv_append + qa_decode_attn at lens = n_past + 1: the whole cache and the
    output bit-exact (new row written, every other row untouched), and the output within the
    attention tolerance of the oracle (which runs the reference order: write the row, then attend)."""
    S = len(n_past)
    lay = layout(qa, 2, S, max(n_past) + 5, f16)
    rng = np.random.default_rng(len(n_past) * 1000 + n_past[0])
    qkv = (rng.standard_normal((S, 4096)) * 0.7).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    d_qkv, d_qn, d_kn = dev(qa, qkv), dev(qa, qn), dev(qa, kn)
    d_np = dev(qa, np.array(n_past, np.int32))
    d_lens = dev(qa, np.array(n_past, np.int32) + 1)
    ws_bytes = qa.lib.qa_decode_attn_workspace_bytes(S, 16, lay.max_seq)
    caches, outs = [], []
    for fused in (True, False):
        cache = Cache(qa, lay)
        cache.fill(np.random.default_rng(99), 1, [p_ + 2 for p_ in n_past])
        ws = zeros(qa, ws_bytes, np.uint8)
        out = zeros(qa, (S, 2048))
        print(f"decode step fused={fused} f16={f16} n_past={n_past}", flush=True)
        if fused:
            qa.check(qa.lib.qa_decode_step_attn(d_qkv.ptr, d_qn.ptr, d_kn.ptr, cache.ptr, C.byref(lay), 1, d_np.ptr, S,
                                                max(n_past) + 1, 16, 1.0e6, 1e-6, SCALE, out.ptr, ws.ptr, ws_bytes,
                                                NULL_STREAM))
        else:
            d_q = zeros(qa, (S, 2048))
            qa.check(qa.lib.qa_kv_append(d_qkv.ptr, d_qn.ptr, d_kn.ptr, d_q.ptr, cache.ptr, C.byref(lay), 1, d_np.ptr,
                                         S, 1, 16, 1.0e6, 1e-6, NULL_STREAM))
            qa.check(qa.lib.qa_decode_attn(d_q.ptr, cache.ptr, C.byref(lay), 1, d_lens.ptr, S, max(n_past) + 1, 16,
                                           SCALE, out.ptr, ws.ptr, ws_bytes, NULL_STREAM))
        qa.synchronize()
        caches.append(cache.read())
        outs.append(out.numpy().reshape(S, 16, 128))
    np.testing.assert_array_equal(caches[0].view(np.uint32), caches[1].view(np.uint32))
    np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    for s_, P in enumerate(n_past):
        k = caches[0][1, 0, s_, :, :P + 1]
        v = caches[0][1, 1, s_, :, :P + 1]
        q, _ = orc.qk_prep(qkv[s_:s_ + 1, :2048].reshape(1, 16, 128), qkv[s_:s_ + 1, 2048:3072].reshape(1, 8, 128),
                           qn, kn, P, 1.0e6, 1e-6)
        ref = orc.cache_attention(k, v, q, P, f16)[0]
        check_close(outs[0][s_], ref)


# ------------------------------------------------------------------------------------------ prefill
@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("n_past,T", [(0, 1), (0, 2), (0, 37), (0, 156), (100, 50), (0, 600), (70, 700), (0, 1024)])
def test_prefill_attention(qa, orc, f16, n_past, T):
    L = n_past + T
    lay = layout(qa, 2, 2, L + 5, f16)
    cache = Cache(qa, lay)
    rng = np.random.default_rng(L)
    vals = cache.fill(rng, 1, [5, L])        # stream 1 holds the rows under test
    k, v = vals[1]
    q = rng.standard_normal((T, 16, 128)).astype(np.float32)
    d_q, d_out = dev(qa, q), zeros(qa, (T, 2048))
    ws_bytes = qa.lib.qa_prefill_attn_workspace_bytes(T, 16)
    ws = zeros(qa, max(ws_bytes, 1), np.uint8)
    print(f"prefill f16={f16} n_past={n_past} T={T}", flush=True)
    qa.check(qa.lib.qa_prefill_attn(d_q.ptr, cache.ptr, C.byref(lay), 1, 1, n_past, T, 16, SCALE, d_out.ptr, ws.ptr,
                                    ws_bytes, NULL_STREAM))
    qa.synchronize()
    got = d_out.numpy().reshape(T, 16, 128)
    ref = orc.cache_attention(k, v, q, n_past, f16)
    check_close(got, ref)
    # row t of the prefill equals a decode over the prefix t + 1 (cross-piece invariant)
    t = T // 2
    dec = orc.cache_attention(k[:, :n_past + t + 1], v[:, :n_past + t + 1], q[t:t + 1], n_past + t, f16)[0]
    check_close(got[t], dec)


@pytest.mark.parametrize("n_past,T", [(0, 3913), (700, 1300)])
def test_prefill_attention_f32_mfma_equals_row_kernel(qa, orc, n_past, T):
    """f32 cache, long prompts: the f32-MFMA kernel (online softmax, exact f32 products) against the f32
    row kernel (QA_PREFILL_F32_ROWS=1, two passes) over every row, and sampled rows against the oracle's
    decode over their prefix."""
    import os

    L = n_past + T
    lay = layout(qa, 2, 1, L + 3, False)
    cache = Cache(qa, lay)
    rng = np.random.default_rng(L + 17)
    k, v = cache.fill(rng, 1, [L])[0]
    q = rng.standard_normal((T, 16, 128)).astype(np.float32)
    d_q = dev(qa, q)
    outs = []
    for rows in ("0", "1"):
        os.environ["QA_PREFILL_F32_ROWS"] = rows
        try:
            d_out = zeros(qa, (T, 2048))
            print(f"prefill f32 rows-kernel={rows} n_past={n_past} T={T}", flush=True)
            qa.check(qa.lib.qa_prefill_attn(d_q.ptr, cache.ptr, C.byref(lay), 1, 0, n_past, T, 16, SCALE, d_out.ptr,
                                            None, 0, NULL_STREAM))
            qa.synchronize()
            outs.append(d_out.numpy().reshape(T, 16, 128))
        finally:
            os.environ.pop("QA_PREFILL_F32_ROWS", None)
    check_close(outs[0], outs[1], atol=2e-5, rtol_l2=2e-6)
    for t in (0, 1, 63, 64, T // 2, T - 1):
        ref = orc.cache_attention(k[:, :n_past + t + 1], v[:, :n_past + t + 1], q[t:t + 1], n_past + t, False)[0]
        check_close(outs[0][t], ref)


@pytest.mark.parametrize("f16", [True, False])
def test_prefill_attention_long_split_rows(qa, orc, f16):
    """Config-3 prefill shape (T = 3913): with an f16 cache the longest query tiles are split over two
    workgroups and merged (f16 MFMA kernel); with an f32 cache the f32-MFMA kernel runs.  Every row of the
    output is held to the oracle's full causal prefill (about 1 s of OpenMP C), each row to the bar on its
    own (2e-3 max-abs, 1e-3 relative L2 over its 16 heads), and sampled rows, in split and unsplit tiles,
    also equal a decode over their prefix."""
    T = 3913
    lay = layout(qa, 1, 1, T + 3, f16)
    cache = Cache(qa, lay)
    rng = np.random.default_rng(T)
    k, v = cache.fill(rng, 0, [T])[0]
    q = rng.standard_normal((T, 16, 128)).astype(np.float32)
    d_q, d_out = dev(qa, q), zeros(qa, (T, 2048))
    ws_bytes = qa.lib.qa_prefill_attn_workspace_bytes(T, 16)
    ws = zeros(qa, max(ws_bytes, 256), np.uint8)
    print(f"prefill split T={T} f16={f16}", flush=True)
    qa.check(qa.lib.qa_prefill_attn(d_q.ptr, cache.ptr, C.byref(lay), 0, 0, 0, T, 16, SCALE, d_out.ptr, ws.ptr,
                                    ws_bytes, NULL_STREAM))
    qa.synchronize()
    got = d_out.numpy().reshape(T, 16, 128).astype(np.float64)
    ref = orc.cache_attention(k, v, q, 0, f16).astype(np.float64)
    err = np.abs(got - ref).reshape(T, -1).max(axis=1)
    rel = np.linalg.norm((got - ref).reshape(T, -1), axis=1) / np.linalg.norm(ref.reshape(T, -1), axis=1)
    worst = int(np.argmax(err))
    print(f"every row: max abs {err.max():.2e} (row {worst}), max rel L2 {rel.max():.2e}", flush=True)
    assert (err <= ATOL).all() and (rel <= RTOL_L2).all(), (worst, err.max(), int(np.argmax(rel)), rel.max())
    for t in (0, 63, 64, 1000, 1983, 1984, 2047, 2048, 3000, 3840, 3841, 3912):
        row = orc.cache_attention(k[:, :t + 1], v[:, :t + 1], q[t:t + 1], t, f16)[0]
        check_close(got[t], row)


_EXACT_PREFILL_CHILD = r"""
import ctypes as C, os, sys
import numpy as np
root = sys.argv[1]
sys.path[:0] = [os.path.join(root, "qwenasr.cpp_amd"), os.path.join(root, "oracle")]
import qwenasr_amd as qa, qa_oracle as orc
scale = 1.0 / np.sqrt(128.0)
for n_past, T in ((0, 5), (0, 300), (600, 700), (0, 3913)):
    L = n_past + T
    lay = qa.KvLayout(1, 1, 8, 128, L + 3, qa.QA_CACHE_F16)
    rng = np.random.default_rng(L + 17)
    host = np.zeros((1, 2, 1, 8, L + 3, 128), np.float16)
    host[0, :, 0, :, :L] = rng.standard_normal((2, 8, L, 128))
    k = host[0, 0, 0, :, :L].astype(np.float32)
    v = host[0, 1, 0, :, :L].astype(np.float32)
    q = rng.standard_normal((T, 16, 128)).astype(np.float32)
    cache, d_q, out = qa.DeviceArray.from_numpy(host), qa.DeviceArray.from_numpy(q), qa.DeviceArray((T, 2048))
    wsb = qa.lib.qa_prefill_attn_workspace_bytes(T, 16)
    ws = qa.DeviceArray(wsb, np.uint8)
    print(f"exact prefill n_past={n_past} T={T}", flush=True)
    qa.check(qa.lib.qa_prefill_attn(d_q.ptr, cache.ptr, C.byref(lay), 0, 0, n_past, T, 16, scale, out.ptr, ws.ptr,
                                    wsb, None))
    got = out.numpy().reshape(T, 16, 128).astype(np.float64)
    ref = orc.cache_attention(k, v, q, n_past, True).astype(np.float64)
    err = np.abs(got - ref).reshape(T, -1).max(axis=1)
    rel = np.linalg.norm((got - ref).reshape(T, -1), axis=1) / np.linalg.norm(ref.reshape(T, -1), axis=1)
    # the two passes round p where the oracle does: an order of magnitude inside the 2e-3 / 1e-3 bar
    assert err.max() <= 2e-4 and rel.max() <= 2e-4, (n_past, T, err.max(), rel.max())
    print(f"  max abs {err.max():.2e}, max rel L2 {rel.max():.2e}", flush=True)
print("exact prefill ok", flush=True)
"""


def test_prefill_attention_exact_two_pass(qa):
    """QA_PREFILL_EXACT=1 (read once per process, so in a child process): the two-pass kernels, which round the
    normalised probabilities to f16 where the reference does, on every row against the oracle at a bar ten times
    tighter than the path's (2e-4), including the config-3 shape with cut tiles and a prefix of cached keys."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, QA_PREFILL_EXACT="1")
    r = subprocess.run([sys.executable, "-c", _EXACT_PREFILL_CHILD, root], env=env, capture_output=True, text=True,
                       timeout=110)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "exact prefill ok" in r.stdout


# fixed region of the prefill workspace: queue counters (4 KB) + 8192 merge counters of 256 bytes
PF_FIXED = 4096 + 8192 * 256


@pytest.mark.parametrize("n_past,T", [(0, 1500), (600, 1500)])
def test_prefill_split_and_unsplit_agree(qa, orc, n_past, T):
    """The longest query tiles cut in two parts (full workspace) and one item per tile (a workspace
    with room for the statistics only) both match the oracle; repeated calls sharing one workspace,
    with other shapes in between, give identical bits (queue and merge counters return to zero)."""
    L = n_past + T
    lay = layout(qa, 1, 1, L + 3, True)
    cache = Cache(qa, lay)
    rng = np.random.default_rng(L + 7)
    k, v = cache.fill(rng, 0, [L])[0]
    q = rng.standard_normal((T, 16, 128)).astype(np.float32)
    d_q = dev(qa, q)
    full = qa.lib.qa_prefill_attn_workspace_bytes(T, 16)
    n_units = (T + 63) // 64 * 8
    small = PF_FIXED + n_units * 2 * 128 * 16         # counters + statistics, no partial outputs
    assert small < full
    ws = zeros(qa, full, np.uint8)
    ref = orc.cache_attention(k, v, q, n_past, True)
    outs = {}
    for label, nbytes in (("split", full), ("unsplit", small), ("split again", full)):
        d_out = zeros(qa, (T, 2048))
        print(f"prefill {label} n_past={n_past} T={T}", flush=True)
        qa.check(qa.lib.qa_prefill_attn(d_q.ptr, cache.ptr, C.byref(lay), 0, 0, n_past, T, 16, SCALE, d_out.ptr,
                                        ws.ptr, nbytes, NULL_STREAM))
        # another shape on the same workspace in between
        d_o2 = zeros(qa, (37, 2048))
        qa.check(qa.lib.qa_prefill_attn(d_q.ptr, cache.ptr, C.byref(lay), 0, 0, 5, 37, 16, SCALE, d_o2.ptr,
                                        ws.ptr, full, NULL_STREAM))
        qa.synchronize()
        outs[label] = d_out.numpy().reshape(T, 16, 128)
        check_close(outs[label], ref)
    np.testing.assert_array_equal(outs["split"].view(np.uint32), outs["split again"].view(np.uint32))
    assert not (ws.numpy()[:PF_FIXED].view(np.uint32)).any(), "queue or merge counters not reset"


def test_prefill_rejects_missing_workspace(qa):
    lay = layout(qa, 1, 1, 70, True)
    cache = Cache(qa, lay)
    d_q, d_out = zeros(qa, (64, 2048)), zeros(qa, (64, 2048))
    rc = qa.lib.qa_prefill_attn(d_q.ptr, cache.ptr, C.byref(lay), 0, 0, 0, 64, 16, SCALE, d_out.ptr, None, 0,
                                NULL_STREAM)
    assert rc != 0


@pytest.mark.parametrize("T", [1, 45, 300])
def test_causal_attention_f32(qa, orc, T):
    rng = np.random.default_rng(T)
    q = rng.standard_normal((T, 16, 128)).astype(np.float32)
    k = rng.standard_normal((T, 8, 128)).astype(np.float32)
    v = rng.standard_normal((T, 8, 128)).astype(np.float32)
    d_q, d_k, d_v, d_o = dev(qa, q), dev(qa, k), dev(qa, v), zeros(qa, (T, 2048))
    qa.check(qa.lib.qa_causal_attn_f32(d_q.ptr, d_k.ptr, d_v.ptr, T, 16, 8, SCALE, d_o.ptr, NULL_STREAM))
    qa.synchronize()
    check_close(d_o.numpy().reshape(T, 16, 128), orc.causal_attention_f32(q, k, v))


# ------------------------------------------------------------------------------------------ adjacent ops
@pytest.mark.parametrize("in_dim", [1024, 2048, 3072, 6144])
@pytest.mark.parametrize("out_dim", [1, 100, 4096])
def test_gemv(qa, orc, in_dim, out_dim):
    rng = np.random.default_rng(in_dim + out_dim)
    w = (rng.standard_normal((out_dim, in_dim)) * 0.02).astype(np.float32)
    x = rng.standard_normal((2, in_dim)).astype(np.float32)
    y0 = rng.standard_normal((2, out_dim)).astype(np.float32)
    d_w, d_x, d_y = dev(qa, w), dev(qa, x), dev(qa, y0)
    qa.check(qa.lib.qa_gemv(d_w.ptr, out_dim, in_dim, d_x.ptr, 2, d_y.ptr, 1, NULL_STREAM))
    qa.synchronize()
    np.testing.assert_allclose(d_y.numpy(), y0 + orc.linear(x, w), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("out_dim,in_dim,rows", [(4096, 2048, 32), (2048, 2048, 5), (12288, 2048, 32),
                                                  (2048, 6144, 32), (20000, 2048, 32), (100, 1024, 64),
                                                  (2048, 6144, 1), (3000, 3072, 17), (4096, 1024, 49),
                                                  (1024, 2048, 49), (6144, 1024, 49), (1024, 3072, 49),
                                                  (1001, 2048, 32), (512, 192, 7), (151936, 256, 32)])
def test_gemm_rows(qa, out_dim, in_dim, rows):
    """Skinny f32 MFMA GEMM of the multi-stream decode step against float64, store and accumulate,
    twice on one workspace (slice counters left at zero)."""
    rng = np.random.default_rng(out_dim + in_dim + rows)
    w = (rng.standard_normal((out_dim, in_dim)) * 0.02).astype(np.float32)
    x = rng.standard_normal((rows, in_dim)).astype(np.float32)
    y0 = rng.standard_normal((rows, out_dim)).astype(np.float32)
    d_w, d_x = dev(qa, w), dev(qa, x)
    wsb = qa.lib.qa_gemm_rows_workspace_bytes(out_dim, in_dim, rows)
    assert wsb > 0
    ws = zeros(qa, wsb, np.uint8)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    print(f"gemm_rows {out_dim}x{in_dim} rows={rows}", flush=True)
    for acc in (0, 1, 0):
        d_y = dev(qa, y0)
        qa.check(qa.lib.qa_gemm_rows(d_w.ptr, out_dim, in_dim, d_x.ptr, rows, d_y.ptr, acc, ws.ptr, wsb, NULL_STREAM))
        qa.synchronize()
        got = d_y.numpy()
        expect = ref + (y0 if acc else 0.0)
        np.testing.assert_allclose(got, expect, rtol=1e-4, atol=2e-4)


def _row_stats(y, n_out):
    """[ceil(n_out / 32)][32] float64 partial sums of squares of each row over 32-column groups."""
    rows = y.shape[0]
    st = np.zeros(((n_out + 31) // 32, 32))
    for k in range(st.shape[0]):
        st[k, :rows] = np.sum(y[:, 32 * k:32 * k + 32].astype(np.float64) ** 2, axis=1)
    return st


@pytest.mark.parametrize("out_dim,in_dim,rows", [(4096, 2048, 32), (2048, 2048, 7), (12288, 2048, 32),
                                                  (2048, 6144, 32), (1056, 1024, 5), (34816, 2048, 32)])
def test_gemm_rows_fused(qa, out_dim, in_dim, rows):
    """Fused skinny GEMM against float64: RMSNorm input from partial sums of squares (the normalised
    row computed in f32 as the RMSNorm kernel does), accumulate + sums of squares of the stored rows,
    and the SwiGLU epilogue over [gate rows; up rows].  34816 rows: more than 1024 tiles of 32 rows (the LM
    head's regime)."""
    rng = np.random.default_rng(out_dim * 3 + in_dim + rows)
    eps = np.float32(1e-6)
    w = (rng.standard_normal((out_dim, in_dim)) * 0.02).astype(np.float32)
    x = rng.standard_normal((rows, in_dim)).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(in_dim)).astype(np.float32)
    y0 = rng.standard_normal((rows, out_dim)).astype(np.float32)
    st_in = _row_stats(x, in_dim)
    # reference normalisation: scale = 1 / sqrtf(float(ss / K) + eps), xn = (x * scale) * w in f32
    ss = np.sum(x.astype(np.float64) ** 2, axis=1)
    scale = (np.float32(1.0) / np.sqrt((ss / in_dim).astype(np.float32) + eps)).astype(np.float32)
    xn = ((x * scale[:, None]).astype(np.float32) * nw[None, :]).astype(np.float32)
    d_w, d_x, d_nw, d_st = dev(qa, w), dev(qa, x), dev(qa, nw), dev(qa, st_in)
    if st_in.shape[0] > 128:        # the RMSNorm input takes at most 128 partials (in_dim <= 4096)
        xn, d_nw, d_st = x, None, None
    wsb = qa.lib.qa_gemm_rows_workspace_bytes(out_dim, in_dim, rows)
    ws = zeros(qa, wsb, np.uint8)
    d_so = zeros(qa, ((out_dim + 31) // 32, 32), np.float64)
    print(f"gemm_rows_fused {out_dim}x{in_dim} rows={rows}", flush=True)
    # RMSNorm input, accumulate, statistics out
    d_y = dev(qa, y0)
    ptr = lambda a: a.ptr if a is not None else None
    qa.check(qa.lib.qa_gemm_rows_fused(d_w.ptr, out_dim, in_dim, d_x.ptr, rows, d_y.ptr, 1, ptr(d_nw), ptr(d_st),
                                       st_in.shape[0], eps, d_so.ptr, 0, ws.ptr, wsb, NULL_STREAM))
    qa.synchronize()
    got = d_y.numpy()
    np.testing.assert_allclose(got, y0 + xn.astype(np.float64) @ w.astype(np.float64).T, rtol=1e-4, atol=2e-4)
    np.testing.assert_allclose(d_so.numpy()[:, :rows], _row_stats(got, out_dim)[:, :rows], rtol=1e-12, atol=0)
    # SwiGLU epilogue: W = [gate; up]
    if out_dim % 32 == 0:
        half = out_dim // 2
        d_a = zeros(qa, (rows, half))
        qa.check(qa.lib.qa_gemm_rows_fused(d_w.ptr, out_dim, in_dim, d_x.ptr, rows, d_a.ptr, 0, ptr(d_nw),
                                           ptr(d_st), st_in.shape[0], eps, None, 1, ws.ptr, wsb, NULL_STREAM))
        qa.synchronize()
        gu = xn.astype(np.float64) @ w.astype(np.float64).T
        g, u = gu[:, :half], gu[:, half:]
        np.testing.assert_allclose(d_a.numpy(), g / (1.0 + np.exp(-g)) * u, rtol=1e-4, atol=2e-4)


def test_gemm_rows_fused_rejects_bad_arguments(qa):
    d = zeros(qa, 1 << 16)
    ws = zeros(qa, qa.lib.qa_gemm_rows_workspace_bytes(64, 1024, 40), np.uint8)
    # more than 32 rows, or an odd SwiGLU split, or no statistics for the RMSNorm input
    assert qa.lib.qa_gemm_rows_fused(d.ptr, 64, 1024, d.ptr, 40, d.ptr, 0, d.ptr, d.ptr, 32, 1e-6, None, 0,
                                     ws.ptr, ws.nbytes, NULL_STREAM) == qa.QA_ERR_INVALID
    assert qa.lib.qa_gemm_rows_fused(d.ptr, 48, 1024, d.ptr, 4, d.ptr, 0, None, None, 0, 0.0, None, 1,
                                     ws.ptr, ws.nbytes, NULL_STREAM) == qa.QA_ERR_INVALID
    assert qa.lib.qa_gemm_rows_fused(d.ptr, 64, 1024, d.ptr, 4, d.ptr, 0, d.ptr, None, 0, 1e-6, None, 0,
                                     ws.ptr, ws.nbytes, NULL_STREAM) == qa.QA_ERR_INVALID


def test_gemm_rows_shared_workspace(qa):
    """One workspace, sized for the largest shape, serves a sequence of different shapes (as in a
    decoder layer) with no clearing: counters and partials never overlap across shapes."""
    rng = np.random.default_rng(11)
    rows = 49
    shapes = [(4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072), (4096, 1024), (6144, 1024)]
    wsb = max(qa.lib.qa_gemm_rows_workspace_bytes(n, k, rows) for n, k in shapes)
    ws = zeros(qa, wsb, np.uint8)
    for n, k in shapes:
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        x = rng.standard_normal((rows, k)).astype(np.float32)
        d_w, d_x, d_y = dev(qa, w), dev(qa, x), zeros(qa, (rows, n))
        print(f"gemm_rows shared {n}x{k}", flush=True)
        qa.check(qa.lib.qa_gemm_rows(d_w.ptr, n, k, d_x.ptr, rows, d_y.ptr, 0, ws.ptr, wsb, NULL_STREAM))
        qa.synchronize()
        np.testing.assert_allclose(d_y.numpy(), x.astype(np.float64) @ w.astype(np.float64).T, rtol=1e-4, atol=2e-4)


def test_gemm_rows_rejects_bad_shapes(qa):
    assert qa.lib.qa_gemm_rows_workspace_bytes(100, 1000, 4) == 0       # in_dim not a multiple of 32
    assert qa.lib.qa_gemm_rows_workspace_bytes(100, 1024, 65) == 0      # more than 64 rows
    d = zeros(qa, 64)
    rc = qa.lib.qa_gemm_rows(d.ptr, 100, 1024, d.ptr, 4, d.ptr, 0, d.ptr, 0, NULL_STREAM)
    assert rc == qa.QA_ERR_INVALID and b"workspace" in qa.lib.qa_last_error()


def test_rmsnorm_rows_bit_exact(qa, orc):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((7, 2048)) * 2).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
    d_x, d_w, d_y = dev(qa, x), dev(qa, w), zeros(qa, (7, 2048))
    qa.check(qa.lib.qa_rmsnorm_rows(d_x.ptr, d_w.ptr, 7, 2048, 1e-6, d_y.ptr, NULL_STREAM))
    qa.synchronize()
    ref = np.stack([orc.rms_norm_row(x[r], w, 1e-6) for r in range(7)])
    np.testing.assert_array_equal(d_y.numpy().view(np.uint32), ref.view(np.uint32))


def test_argmax_rows_rule(qa, orc):
    V = 151936
    rng = np.random.default_rng(4)
    rows = [rng.standard_normal(V).astype(np.float32) for _ in range(3)]
    rows[1][[5, 90000, 151935]] = 50.0                         # ties: first index wins
    rows[2][:] = np.nan
    rows[2][77777] = -3.0                                      # NaN never wins
    rows.append(np.full(V, -np.inf, np.float32))               # nothing beats -inf -> -1
    logits = np.stack(rows)
    d_l, d_ids = dev(qa, logits), zeros(qa, 4, np.int32)
    ws_bytes = qa.lib.qa_argmax_workspace_bytes(4)
    ws = zeros(qa, ws_bytes, np.uint8)
    for _ in range(2):
        qa.check(qa.lib.qa_argmax_rows(d_l.ptr, 4, V, d_ids.ptr, ws.ptr, ws_bytes, NULL_STREAM))
        qa.synchronize()
        assert d_ids.numpy().tolist() == [orc.argmax(r) for r in rows] == [int(np.argmax(rows[0])), 5, 77777, -1]


@pytest.mark.parametrize("V", [151936, 200000, 1000])
def test_argmax_ties_within_one_thread(qa, orc, V):
    """Each thread scans its elements (256 apart) in batches of loads; ties between elements of one thread, in
    one batch and across batches (V = 200000: 13 elements per thread), keep the lowest index, and a larger value
    in a later batch still wins.  V = 1000: most threads have no element (clamped loads are skipped)."""
    rng = np.random.default_rng(V)
    chunk = (V + 63) // 64
    base = 3 * chunk + 7                                        # thread 7 of block 3
    a = rng.standard_normal(V).astype(np.float32)
    b = rng.standard_normal(V).astype(np.float32)
    if V >= 100000:
        a[[base, base + 256 * 4]] = 40.0                        # one batch
        b[[base + 256 * 2, base + 256 * 11 if V > 160000 else base + 256 * 9]] = [40.0, 41.0]
        want = [base, base + 256 * 11 if V > 160000 else base + 256 * 9]
    else:
        a[[3, 700]] = 40.0
        b[999] = 40.0
        want = [3, 999]
    d_l, d_ids = dev(qa, np.stack([a, b])), zeros(qa, 2, np.int32)
    ws_bytes = qa.lib.qa_argmax_workspace_bytes(2)
    ws = zeros(qa, ws_bytes, np.uint8)
    qa.check(qa.lib.qa_argmax_rows(d_l.ptr, 2, V, d_ids.ptr, ws.ptr, ws_bytes, NULL_STREAM))
    qa.synchronize()
    assert d_ids.numpy().tolist() == [orc.argmax(a), orc.argmax(b)] == want


def test_embed_and_lens(qa):
    table = np.arange(10 * 2048, dtype=np.float32).reshape(10, 2048)
    d_t, d_ids = dev(qa, table), dev(qa, np.array([3, -1, 9, 10], np.int32))
    d_o = dev(qa, np.ones((4, 2048), np.float32))
    qa.check(qa.lib.qa_embed_rows(d_t.ptr, 10, 2048, d_ids.ptr, 4, d_o.ptr, NULL_STREAM))
    d_lens = dev(qa, np.array([0, 5, 7], np.int32))
    qa.check(qa.lib.qa_advance_lens(d_lens.ptr, 3, 2, NULL_STREAM))
    qa.synchronize()
    o = d_o.numpy()
    np.testing.assert_array_equal(o[0], table[3])
    np.testing.assert_array_equal(o[2], table[9])
    assert not o[1].any() and not o[3].any()
    assert d_lens.numpy().tolist() == [2, 7, 9]


def test_event_timing_helpers(qa):
    """The C-ABI event pair measures a positive interval around device work."""
    a, b = C.c_void_p(), C.c_void_p()
    qa.check(qa.lib.qa_event_create(C.byref(a)))
    qa.check(qa.lib.qa_event_create(C.byref(b)))
    x = zeros(qa, (1 << 20,))
    qa.check(qa.lib.qa_event_record(a, NULL_STREAM))
    for _ in range(10):
        qa.check(qa.lib.qa_add_inplace(x.ptr, x.ptr, 1 << 20, NULL_STREAM))
    qa.check(qa.lib.qa_event_record(b, NULL_STREAM))
    ms = C.c_float()
    qa.check(qa.lib.qa_event_elapsed_ms(a, b, C.byref(ms)))
    assert ms.value > 0.0
    qa.check(qa.lib.qa_event_destroy(a))
    qa.check(qa.lib.qa_event_destroy(b))
