"""Kernel-level parity of the HIP path against the CPU oracle, through the C ABI.

Device memory comes from torch (plumbing only); every computation is a qa_* entry point of
libqwenasr_amd.so.  Bars: cache slots, positions and lengths bit-exact;
attention within 2e-3 max-abs and 1e-3 relative-L2 with f32 accumulation.  The append kernel is
held to bit-exactness of the whole cache (written rows and untouched rows alike).
"""
import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

ATOL, RTOL_L2 = 2e-3, 1e-3


def vp(t):
    return C.c_void_p(t.data_ptr())


def stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


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


def layout(qa, n_layers, n_streams, max_seq, f16):
    return qa.KvLayout(n_layers, n_streams, 8, 128, max_seq, qa.QA_CACHE_F16 if f16 else qa.QA_CACHE_F32)


def cache_tensor(qa, lay):
    n = qa.lib.qa_kv_cache_bytes(C.byref(lay))
    return torch.zeros(n // (2 if lay.cache_type == qa.QA_CACHE_F16 else 4),
                       dtype=torch.float16 if lay.cache_type == qa.QA_CACHE_F16 else torch.float32, device="cuda")


def cache_view(lay, t):
    """[layer][kv][stream][head][pos][dim] numpy view of the device cache (as f32 values)."""
    a = t.cpu().numpy().astype(np.float32)
    return a.reshape(lay.n_layers, 2, lay.n_streams, lay.n_kv_heads, lay.max_seq, lay.head_dim)


# ------------------------------------------------------------------------------------------ append
@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("T,n_past", [(1, [0, 17, 4167]), (5, [3, 100, 4000]), (156, [0])])
def test_kv_append_bit_exact(qa, orc, f16, T, n_past):
    S = len(n_past)
    lay = layout(qa, 2, S, 4169, f16)
    cache = cache_tensor(qa, lay)
    rng = np.random.default_rng(T * 7 + S)
    qkv = (rng.standard_normal((S * T, 4096)) * 0.7).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    d_qkv, d_qn, d_kn = dev(qkv), dev(qn), dev(kn)
    d_q = torch.zeros(S * T, 2048, device="cuda")
    d_np = dev(np.array(n_past, np.int32))
    print(f"append f16={f16} T={T} n_past={n_past}", flush=True)
    qa.check(qa.lib.qa_kv_append(vp(d_qkv), vp(d_qn), vp(d_kn), vp(d_q), vp(cache), C.byref(lay), 1, vp(d_np), S, T,
                                 16, 1.0e6, 1e-6, stream()))
    torch.cuda.synchronize()
    got = cache_view(lay, cache)
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
        np.testing.assert_array_equal(d_q[s * T:(s + 1) * T].cpu().numpy().view(np.uint32),
                                      q.reshape(T, 2048).view(np.uint32))
    np.testing.assert_array_equal(got.view(np.uint32), expect.view(np.uint32))


# ------------------------------------------------------------------------------------------ decode
def _fill_cache(qa, lay, cache, rng, layer, stream_lens):
    """Random K/V rows [0, L) per stream at `layer`; returns the f32 values actually stored."""
    vals = {}
    full = cache.view(lay.n_layers, 2, lay.n_streams, lay.n_kv_heads, lay.max_seq, lay.head_dim)
    for s, L in enumerate(stream_lens):
        k = rng.standard_normal((8, L, 128)).astype(np.float32)
        v = rng.standard_normal((8, L, 128)).astype(np.float32)
        full[layer, 0, s, :, :L] = torch.from_numpy(k).to(full.dtype)
        full[layer, 1, s, :, :L] = torch.from_numpy(v).to(full.dtype)
        vals[s] = (k, v)
    return vals


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("lens", [[1], [2], [63], [64], [65], [157], [1000], [4096], [156, 3913, 700, 1, 2048]])
def test_decode_attention(qa, orc, f16, lens):
    S = len(lens)
    max_len = max(lens)
    lay = layout(qa, 3, S, max_len + 3, f16)
    cache = cache_tensor(qa, lay)
    rng = np.random.default_rng(sum(lens))
    vals = _fill_cache(qa, lay, cache, rng, 2, lens)
    q = rng.standard_normal((S, 16, 128)).astype(np.float32)
    d_q, d_out = dev(q), torch.zeros(S, 2048, device="cuda")
    d_lens = dev(np.array(lens, np.int32))
    ws_bytes = qa.lib.qa_decode_attn_workspace_bytes(S, 16, max_len)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device="cuda")
    print(f"decode f16={f16} lens={lens}", flush=True)
    for rep in range(2):   # the second call checks the counters were left at zero
        qa.check(qa.lib.qa_decode_attn(vp(d_q), vp(cache), C.byref(lay), 2, vp(d_lens), S, max_len, 16,
                                       1.0 / np.sqrt(128.0), vp(d_out), vp(ws), ws_bytes, stream()))
        torch.cuda.synchronize()
        got = d_out.cpu().numpy().reshape(S, 16, 128)
        for s, L in enumerate(lens):
            k, v = vals[s]
            ref = orc.cache_attention(k, v, q[s:s + 1], L - 1, f16)[0]
            check_close(got[s], ref)


# ------------------------------------------------------------------------------------------ prefill
@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("n_past,T", [(0, 1), (0, 2), (0, 37), (0, 156), (100, 50), (0, 600)])
def test_prefill_attention(qa, orc, f16, n_past, T):
    L = n_past + T
    lay = layout(qa, 2, 2, L + 5, f16)
    cache = cache_tensor(qa, lay)
    rng = np.random.default_rng(L)
    vals = _fill_cache(qa, lay, cache, rng, 1, [5, L])        # stream 1 holds the rows under test
    k, v = vals[1]
    q = rng.standard_normal((T, 16, 128)).astype(np.float32)
    d_q, d_out = dev(q), torch.zeros(T, 2048, device="cuda")
    ws_bytes = qa.lib.qa_prefill_attn_workspace_bytes(T, 16)
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    print(f"prefill f16={f16} n_past={n_past} T={T}", flush=True)
    qa.check(qa.lib.qa_prefill_attn(vp(d_q), vp(cache), C.byref(lay), 1, 1, n_past, T, 16, 1.0 / np.sqrt(128.0),
                                    vp(d_out), vp(ws), ws_bytes, stream()))
    torch.cuda.synchronize()
    got = d_out.cpu().numpy().reshape(T, 16, 128)
    ref = orc.cache_attention(k, v, q, n_past, f16)
    check_close(got, ref)
    # row t of the prefill equals a decode over the prefix t + 1 (cross-piece invariant)
    t = T // 2
    dec = orc.cache_attention(k[:, :n_past + t + 1], v[:, :n_past + t + 1], q[t:t + 1], n_past + t, f16)[0]
    check_close(got[t], dec)


@pytest.mark.parametrize("T", [1, 45, 300])
def test_causal_attention_f32(qa, orc, T):
    rng = np.random.default_rng(T)
    q = rng.standard_normal((T, 16, 128)).astype(np.float32)
    k = rng.standard_normal((T, 8, 128)).astype(np.float32)
    v = rng.standard_normal((T, 8, 128)).astype(np.float32)
    d_q, d_k, d_v, d_o = dev(q), dev(k), dev(v), torch.zeros(T, 2048, device="cuda")
    qa.check(qa.lib.qa_causal_attn_f32(vp(d_q), vp(d_k), vp(d_v), T, 16, 8, 1.0 / np.sqrt(128.0), vp(d_o), stream()))
    torch.cuda.synchronize()
    check_close(d_o.cpu().numpy().reshape(T, 16, 128), orc.causal_attention_f32(q, k, v))


# ------------------------------------------------------------------------------------------ adjacent ops
@pytest.mark.parametrize("in_dim", [1024, 2048, 3072, 6144])
@pytest.mark.parametrize("out_dim", [1, 100, 4096])
def test_gemv(qa, orc, in_dim, out_dim):
    rng = np.random.default_rng(in_dim + out_dim)
    w = (rng.standard_normal((out_dim, in_dim)) * 0.02).astype(np.float32)
    x = rng.standard_normal((2, in_dim)).astype(np.float32)
    y0 = rng.standard_normal((2, out_dim)).astype(np.float32)
    d_w, d_x, d_y = dev(w), dev(x), dev(y0)
    qa.check(qa.lib.qa_gemv(vp(d_w), out_dim, in_dim, vp(d_x), 2, vp(d_y), 1, stream()))
    torch.cuda.synchronize()
    np.testing.assert_allclose(d_y.cpu().numpy(), y0 + orc.linear(x, w), rtol=1e-5, atol=1e-5)


def test_rmsnorm_rows_bit_exact(qa, orc):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((7, 2048)) * 2).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
    d_x, d_w, d_y = dev(x), dev(w), torch.zeros(7, 2048, device="cuda")
    qa.check(qa.lib.qa_rmsnorm_rows(vp(d_x), vp(d_w), 7, 2048, 1e-6, vp(d_y), stream()))
    torch.cuda.synchronize()
    ref = np.stack([orc.rms_norm_row(x[r], w, 1e-6) for r in range(7)])
    np.testing.assert_array_equal(d_y.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_argmax_rows_rule(qa, orc):
    V = 151936
    rng = np.random.default_rng(4)
    rows = [rng.standard_normal(V).astype(np.float32) for _ in range(3)]
    rows[1][[5, 90000, 151935]] = 50.0                         # ties: first index wins
    rows[2][:] = np.nan
    rows[2][77777] = -3.0                                      # NaN never wins
    rows.append(np.full(V, -np.inf, np.float32))               # nothing beats -inf -> -1
    logits = np.stack(rows)
    d_l, d_ids = dev(logits), torch.zeros(4, dtype=torch.int32, device="cuda")
    ws_bytes = qa.lib.qa_argmax_workspace_bytes(4)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device="cuda")
    for _ in range(2):
        qa.check(qa.lib.qa_argmax_rows(vp(d_l), 4, V, vp(d_ids), vp(ws), ws_bytes, stream()))
        torch.cuda.synchronize()
        assert d_ids.cpu().tolist() == [orc.argmax(r) for r in rows] == [int(np.argmax(rows[0])), 5, 77777, -1]


def test_embed_and_lens(qa):
    table = np.arange(10 * 2048, dtype=np.float32).reshape(10, 2048)
    d_t, d_ids, d_o = dev(table), dev(np.array([3, -1, 9, 10], np.int32)), torch.ones(4, 2048, device="cuda")
    qa.check(qa.lib.qa_embed_rows(vp(d_t), 10, 2048, vp(d_ids), 4, vp(d_o), stream()))
    d_lens = dev(np.array([0, 5, 7], np.int32))
    qa.check(qa.lib.qa_advance_lens(vp(d_lens), 3, 2, stream()))
    torch.cuda.synchronize()
    o = d_o.cpu().numpy()
    np.testing.assert_array_equal(o[0], table[3])
    np.testing.assert_array_equal(o[2], table[9])
    assert not o[1].any() and not o[3].any()
    assert d_lens.cpu().tolist() == [2, 7, 9]
