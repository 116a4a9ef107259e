"""bf16-exact weights on the GPU: the decoder's bf16 weight copies give the f32 results bit for bit.

A checkpoint converted from the released bf16 weights (convert.py:386-387 widens each bf16 tensor
with tensor.float()) holds f32 values with zero low halves.  The decoder then keeps bf16 copies of
its projection and LM-head weights and the batch-1 GEMVs widen them back in registers.  These tests
hold that path to bit-equality with the f32 GEMV on the same values (every epilogue, every input
width), to a float64 restatement of the GEMV, and, end to end, to the f32-storage decoder and the
oracle's greedy ids."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu(qa):
    assert qa.device_count() > 0, "no HIP device: GPU tests need the MI355X"


def bf16_round(a):
    """Nearest bf16 value (ties to even) of each f32, as f32 (torch's own conversion)."""
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


def high_halves(a):
    return (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def gemv_f64(w, x, epilogue, norm_w, eps, y0):
    x = x.astype(np.float64)
    if norm_w is not None:
        x32 = x.astype(np.float32)
        scale = np.float32(1.0) / np.sqrt(np.float32(np.sum(x * x) / x.size) + np.float32(eps))
        x = ((x32 * scale) * norm_w).astype(np.float64)
    if epilogue == 2:
        n = w.shape[0] // 2
        g, u = w[:n].astype(np.float64) @ x, w[n:].astype(np.float64) @ x
        return g / (1.0 + np.exp(-g)) * u
    y = w.astype(np.float64) @ x
    return y + y0 if epilogue == 1 else y


def run_gemv(qa, w, x, epilogue, norm_w, y0, b16):
    out_dim = w.shape[0] // 2 if epilogue == 2 else w.shape[0]
    d_x = qa.DeviceArray.from_numpy(x)
    d_y = qa.DeviceArray.from_numpy(y0.copy())
    d_n = qa.DeviceArray.from_numpy(norm_w) if norm_w is not None else None
    if b16:
        d_w = qa.DeviceArray.from_numpy(high_halves(w))
        args = (None, d_w.ptr)
    else:
        d_w = qa.DeviceArray.from_numpy(w)
        args = (d_w.ptr, None)
    qa.check(qa.lib.qa_gemv_fused(*args, out_dim, w.shape[1], d_x.ptr, d_y.ptr, epilogue,
                                  d_n.ptr if d_n is not None else None, 1e-6, None))
    qa.synchronize()
    return d_y.numpy()


@pytest.mark.parametrize("in_dim", [1024, 2048, 3072, 4096, 6144])
@pytest.mark.parametrize("epilogue,prenorm", [(0, False), (0, True), (1, False), (2, True)])
@pytest.mark.parametrize("out_dim", [1, 100, 4096])
def test_gemv_bf16_copy_equals_f32_bit_for_bit(qa, in_dim, epilogue, prenorm, out_dim):
    rng = np.random.default_rng(in_dim * 7 + out_dim + epilogue)
    rows = 2 * out_dim if epilogue == 2 else out_dim
    w = bf16_round(rng.standard_normal((rows, in_dim)) * 0.02)
    assert not (w.view(np.uint32) & 0xffff).any()
    x = rng.standard_normal(in_dim).astype(np.float32)
    norm_w = (1.0 + 0.1 * rng.standard_normal(in_dim)).astype(np.float32) if prenorm else None
    y0 = rng.standard_normal(out_dim).astype(np.float32)
    y32 = run_gemv(qa, w, x, epilogue, norm_w, y0, False)
    y16 = run_gemv(qa, w, x, epilogue, norm_w, y0, True)
    np.testing.assert_array_equal(y16.view(np.uint32), y32.view(np.uint32))
    np.testing.assert_allclose(y16, gemv_f64(w, x, epilogue, norm_w, 1e-6, y0), rtol=2e-5, atol=2e-5)


def test_gemv_fused_rejects_ambiguous_weights(qa):
    d = qa.DeviceArray((64,), np.float32)
    for args in ((None, None), (d.ptr, d.ptr)):
        with pytest.raises(qa.QaError) as e:
            qa.check(qa.lib.qa_gemv_fused(*args, 4, 1024, d.ptr, d.ptr, 0, None, 1e-6, None))
        assert e.value.code == qa.QA_ERR_INVALID
    with pytest.raises(qa.QaError):
        qa.check(qa.lib.qa_gemv_fused(d.ptr, None, 4, 1000, d.ptr, d.ptr, 0, None, 1e-6, None))


@pytest.mark.parametrize("n", [1, 255, 4096, 1000003])
def test_pack_bf16_flags_inexact_values(qa, n):
    rng = np.random.default_rng(n)
    a = bf16_round(rng.standard_normal(n))
    flag = qa.DeviceArray((1,), np.uint32)
    d_a = qa.DeviceArray.from_numpy(a)
    d_b = qa.DeviceArray((n,), np.uint16)
    qa.check(qa.lib.qa_pack_bf16(d_a.ptr, n, d_b.ptr, flag.ptr, None))
    qa.synchronize()
    assert int(flag.numpy()[0]) == 0
    np.testing.assert_array_equal(d_b.numpy(), high_halves(a))
    b = a.copy()
    b.view(np.uint32)[n // 2] |= 1           # one value with a non-zero low half
    d_a.upload(b)
    qa.check(qa.lib.qa_pack_bf16(d_a.ptr, n, d_b.ptr, flag.ptr, None))
    qa.synchronize()
    assert int(flag.numpy()[0]) == 1


def _decoder(qa, model, max_seq, f32_weights):
    """A decoder created with QA_WEIGHTS_F32=1 (f32_weights), which is read at creation, so the environment
    is restored right after."""
    saved = {k: os.environ.pop(k, None) for k in ("QA_WEIGHTS_F32",)}
    try:
        if f32_weights:
            os.environ["QA_WEIGHTS_F32"] = "1"
        return qa.Decoder(model, 1, max_seq, qa.QA_CACHE_F16)
    finally:
        for k, v in saved.items():
            os.environ.pop(k, None)
            if v is not None:
                os.environ[k] = v


def test_decoder_keeps_bf16_copies_only_for_exact_weights(qa):
    exact = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=2, bf16=True)
    plain = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=2)
    with _decoder(qa, exact, 64, False) as d:
        assert d.weights_bf16
    with _decoder(qa, exact, 64, True) as d:
        assert not d.weights_bf16
    with _decoder(qa, plain, 64, False) as d:
        assert not d.weights_bf16          # N(0, 0.02) draws are not bf16 values


def test_bf16_weights_generate_equals_f32_weights_and_oracle(qa, orc, greedy):
    """0.6B shapes, 3 layers, bf16-exact weights: the bf16-copy decoder and the f32 decoder produce
    bit-identical logits and identical ids; both match the oracle's greedy ids."""
    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=3, bf16=True)
    om = orc.OracleModel.from_product_model(model)
    x = qa.prompt_input(model, 40, 9)
    N = 24
    ref = om.generate(x, N, qa.STOP_IDS, om.cache(49 + N, True))
    outs, logits = [], []
    for f32_weights in (False, True):
        with _decoder(qa, model, 49 + N, f32_weights) as dec:
            assert dec.weights_bf16 == (not f32_weights)
            outs.append(dec.generate(x, N, margins=True))
            logits.append(dec.forward(x, 0))
    assert outs[0] == outs[1]
    np.testing.assert_array_equal(logits[0].view(np.uint32), logits[1].view(np.uint32))
    assert greedy.match(outs[0]["ids"], ref["ids"], ref["margins"], ref["runner_up"],
                        "bf16-exact weights, 0.6B x 3 layers") is None


def _row_stats(x, dim):
    n = (dim + 31) // 32
    st = np.zeros((n, 32), np.float64)
    for k in range(n):
        st[k, :x.shape[0]] = np.sum(x[:, 32 * k:32 * k + 32].astype(np.float64) ** 2, axis=1)
    return st


@pytest.mark.parametrize("out_dim,in_dim,rows", [(4096, 2048, 32), (2048, 2048, 7), (12288, 2048, 32),
                                                  (2048, 6144, 32), (1056, 1024, 5), (151936 // 8, 2048, 32)])
def test_gemm_rows_bf16_matches_float64(qa, out_dim, in_dim, rows):
    """The multi-stream step's 32-row GEMM on bf16 weights (bf16 MFMAs over x split into three bf16
    parts: exact products, f32 sums) against float64 of the same f32 inputs, with each fusion: RMSNorm
    input + accumulate + statistics out, and the SwiGLU epilogue.  The bar is about ten times the f32
    accumulation error of these sums; the f32-weight kernel meets the same bar on the same inputs."""
    rng = np.random.default_rng(out_dim + in_dim + rows)
    eps = np.float32(1e-6)
    w = bf16_round(rng.standard_normal((out_dim, in_dim)) * 0.02)
    x = rng.standard_normal((rows, in_dim)).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(in_dim)).astype(np.float32)
    y0 = rng.standard_normal((rows, out_dim)).astype(np.float32)
    st_in = _row_stats(x, in_dim)
    d_x = qa.DeviceArray.from_numpy(x)
    norm = st_in.shape[0] <= 128
    d_nw = qa.DeviceArray.from_numpy(nw) if norm else None
    d_st = qa.DeviceArray.from_numpy(st_in) if norm else None
    # the normalised input as both kernels form it: scale = 1 / sqrtf(float(ss / K) + eps), (x * scale) * w
    if norm:
        ss = np.sum(x.astype(np.float64) ** 2, axis=1)
        scale = (np.float32(1.0) / np.sqrt((ss / in_dim).astype(np.float32) + eps)).astype(np.float32)
        xn = ((x * scale[:, None]).astype(np.float32) * nw[None, :]).astype(np.float32)
    else:
        xn = x
    ref = xn.astype(np.float64) @ w.T.astype(np.float64)
    wsb = qa.lib.qa_gemm_rows_workspace_bytes(out_dim, in_dim, rows)
    ws = qa.DeviceArray((wsb,), np.uint8)
    d_w32 = qa.DeviceArray.from_numpy(w)
    d_w16 = qa.DeviceArray.from_numpy(high_halves(w))
    ptr = lambda a: a.ptr if a is not None else None
    print(f"gemm_rows bf16 {out_dim}x{in_dim} rows={rows}", flush=True)
    for fn, d_w in ((qa.lib.qa_gemm_rows_fused, d_w32), (qa.lib.qa_gemm_rows_fused_bf16, d_w16)):
        d_y = qa.DeviceArray.from_numpy(y0)
        d_so = qa.DeviceArray(((out_dim + 31) // 32, 32), np.float64)
        qa.check(fn(d_w.ptr, out_dim, in_dim, d_x.ptr, rows, d_y.ptr, 1, ptr(d_nw), ptr(d_st), st_in.shape[0],
                    eps, d_so.ptr, 0, ws.ptr, wsb, None))
        qa.synchronize()
        y = d_y.numpy()
        np.testing.assert_allclose(y, y0 + ref, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(d_so.numpy()[:, :rows], _row_stats(y, out_dim)[:, :rows], rtol=1e-12, atol=0)
        if out_dim % 32 == 0:
            half = out_dim // 2
            d_a = qa.DeviceArray((rows, half), np.float32)
            qa.check(fn(d_w.ptr, out_dim, in_dim, d_x.ptr, rows, d_a.ptr, 0, ptr(d_nw), ptr(d_st), st_in.shape[0],
                        eps, None, 1, ws.ptr, wsb, None))
            qa.synchronize()
            g, u = ref[:, :half], ref[:, half:]
            np.testing.assert_allclose(d_a.numpy(), g / (1.0 + np.exp(-g)) * u, rtol=1e-5, atol=1e-5)


def test_gemm_rows_bf16_rejects_unsupported_shapes(qa):
    d = qa.DeviceArray((1 << 16,), np.float32)
    ws = qa.DeviceArray((1 << 20,), np.uint8)
    with pytest.raises(qa.QaError) as e:       # 33 rows take the longer-row kernel, which reads f32 weights
        qa.check(qa.lib.qa_gemm_rows_fused_bf16(d.ptr, 64, 64, d.ptr, 33, d.ptr, 0, None, None, 0, 1e-6, None, 0,
                                                ws.ptr, 1 << 20, None))
    assert e.value.code == qa.QA_ERR_INVALID
    with pytest.raises(qa.QaError):
        qa.check(qa.lib.qa_gemm_rows_fused_bf16(None, 64, 64, d.ptr, 4, d.ptr, 0, None, None, 0, 1e-6, None, 0,
                                                ws.ptr, 1 << 20, None))


def split3(a):
    """The exact three-part bf16 split of f32 values (a = hi + mid + lo), as bf16 bits [hi, mid, lo]."""
    a = np.ascontiguousarray(a, np.float32)
    hi = (a.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    r1 = (a - hi).astype(np.float32)
    mid = (r1.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    lo = (r1 - mid).astype(np.float32)
    assert np.array_equal((hi + mid) + lo, a)
    return [high_halves(v) for v in (hi, mid, lo)]


@pytest.mark.parametrize("rows,out_dim,in_dim,mode", [
    (1, 256, 64, "store"), (73, 2048, 2048, "accumulate"), (300, 4096, 2048, "store"), (200, 1024, 3072, "swiglu"),
    (300, 768, 128, "accumulate"), (129, 384, 192, "swiglu"),
    (3913, 4096, 2048, "store"), (3913, 2048, 6144, "accumulate"), (3913, 6144, 2048, "swiglu")])
def test_gemm_split3_bf16_matches_float64(qa, rows, out_dim, in_dim, mode):
    """The prefill GEMM on bf16-exact weights (rows > 32): bf16 MFMAs over the three-part split of each
    input row against the one bf16 copy of W, every product exact, sums in f32.  Against float64 of the same
    f32 inputs, at the 1.7B prefill shapes (T = 3913: q|k|v, down, gate|up) and at ragged row counts (the
    last 128-row tile partly filled; 1 row); 768 and 384 output columns split into 3 column tiles, which take
    the plain tile order instead of the per-XCD one.  Store, accumulate (the residual add of o and down) and the
    SwiGLU epilogue, which writes the split of silu(gate) * up: its parts are checked bit for bit against
    the split of the kernel's own values, and the values against float64."""
    rng = np.random.default_rng(rows + out_dim + in_dim)
    n_w = 2 * out_dim if mode == "swiglu" else out_dim
    w = bf16_round(rng.standard_normal((n_w, in_dim)) * 0.02)
    x = rng.standard_normal((rows, in_dim)).astype(np.float32)
    xs = np.concatenate(split3(x), axis=1)                      # [rows][3 in_dim]
    ref = x.astype(np.float64) @ w.T.astype(np.float64)
    d_w = qa.DeviceArray.from_numpy(high_halves(w))
    d_xs = qa.DeviceArray.from_numpy(xs)
    print(f"gemm_split3 rows={rows} {out_dim}x{in_dim} {mode}", flush=True)
    if mode == "swiglu":
        d_a = qa.DeviceArray.from_numpy(np.zeros((rows, 3 * out_dim), np.uint16))
        qa.check(qa.lib.qa_gemm_split3_bf16(d_w.ptr, out_dim, in_dim, d_xs.ptr, rows, None, 0, d_a.ptr, None))
        qa.synchronize()
        a = d_a.numpy()
        parts = [(a[:, p * out_dim:(p + 1) * out_dim].astype(np.uint32) << 16).view(np.float32) for p in range(3)]
        v = (parts[0] + parts[1]) + parts[2]
        assert all(np.array_equal(got, want) for got, want in
                   zip((a[:, p * out_dim:(p + 1) * out_dim] for p in range(3)), split3(v)))
        g, u = ref[:, :out_dim], ref[:, out_dim:]
        np.testing.assert_allclose(v, g / (1.0 + np.exp(-g)) * u, rtol=1e-5, atol=1e-5)
        return
    y0 = rng.standard_normal((rows, out_dim)).astype(np.float32)
    d_y = qa.DeviceArray.from_numpy(y0 if mode == "accumulate" else np.zeros_like(y0))
    qa.check(qa.lib.qa_gemm_split3_bf16(d_w.ptr, out_dim, in_dim, d_xs.ptr, rows, d_y.ptr,
                                        int(mode == "accumulate"), None, None))
    qa.synchronize()
    want = ref + y0 if mode == "accumulate" else ref
    np.testing.assert_allclose(d_y.numpy(), want, rtol=1e-5, atol=1e-5)


def test_gemm_split3_bf16_rejects_unsupported_shapes(qa):
    d = qa.DeviceArray((1 << 16,), np.float32)
    for args in ((d.ptr, 300, 64, d.ptr, 130, d.ptr, 0, None),      # out_dim % 256
                 (d.ptr, 256, 96, d.ptr, 130, d.ptr, 0, None),      # in_dim % 64
                 (None, 256, 64, d.ptr, 130, d.ptr, 0, None),       # no weights
                 (d.ptr, 256, 64, d.ptr, 0, d.ptr, 0, None),        # no rows
                 (d.ptr, 256, 64, d.ptr, 130, d.ptr, 0, d.ptr),     # SwiGLU writes the split, not y
                 (d.ptr, 192, 64, d.ptr, 130, None, 0, d.ptr)):     # SwiGLU: out_dim % 128
        with pytest.raises(qa.QaError) as e:
            qa.check(qa.lib.qa_gemm_split3_bf16(*args, None))
        assert e.value.code == qa.QA_ERR_INVALID


@pytest.mark.parametrize("n_streams", [5, 32])
def test_bf16_weights_multistream_equals_f32_weights_and_oracle(qa, orc, greedy, n_streams):
    """The multi-stream decode step with bf16-exact weights: the bf16-copy decoder (bf16 MFMAs) and the
    f32 decoder both match the oracle decoding each stream alone (0.6B, 2 layers)."""
    from qwenasr_amd import configs

    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=2, bf16=True)
    om = orc.OracleModel.from_product_model(model)
    rng = np.random.default_rng(100 + n_streams)
    lens = rng.integers(20, 180, n_streams)
    first = rng.integers(0, model.cfg.vocab, n_streams).astype(np.int32)
    steps, cap = 4, 200
    kv = [configs.cfg4_stream_kv(2000 + s, int(lens[s]), n_layers=2) for s in range(n_streams)]
    got = []
    for f32_weights in (False, True):
        old = os.environ.pop("QA_WEIGHTS_F32", None)
        if f32_weights:
            os.environ["QA_WEIGHTS_F32"] = "1"
        try:
            dec = qa.Decoder(model, n_streams, cap, qa.QA_CACHE_F16)
        finally:
            os.environ.pop("QA_WEIGHTS_F32", None)
            if old is not None:
                os.environ["QA_WEIGHTS_F32"] = old
        with dec:
            assert dec.weights_bf16 == (not f32_weights)
            for s in range(n_streams):
                dec.fill_cache(s, kv[s][0], kv[s][1], int(lens[s]))
            got.append(dec.decode_streams(first, steps))
    for s in range(n_streams):
        cache = om.cache(cap, True)
        cache.fill(kv[s][0], kv[s][1], int(lens[s]))
        ids, margins, runner = om.decode_steps(cache, int(first[s]), steps)
        for g, name in zip(got, ("bf16 copies", "f32 weights")):
            greedy.match(g[:, s].tolist(), list(ids), list(margins), list(runner),
                         f"bf16-exact weights ({name}), {n_streams}-stream step, stream {s}")


def test_bf16_weights_long_prefill_matches_oracle(qa, orc, greedy):
    """A 300-position prompt (longer than the 64 rows of the skinny GEMM): with bf16 copies each prefill
    projection is one bf16 MFMA GEMM (gemm_split3) over the exact three-part split of its input and the one
    bf16 copy of the weights, gate|up with the SwiGLU fused (exact products, f32 sums).  Logits against the
    oracle and against the f32-weight decoder, then greedy ids."""
    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=3, bf16=True)
    om = orc.OracleModel.from_product_model(model)
    x = qa.prompt_input(model, 290, 10)
    N = 16
    ref_logits = om.forward_cached(x, 0, om.cache(300 + N, True))
    ref = om.generate(x, N, qa.STOP_IDS, om.cache(300 + N, True))
    logits = {}
    for f32_weights in (False, True):
        with _decoder(qa, model, 300 + N, f32_weights) as dec:
            assert dec.weights_bf16 == (not f32_weights)
            logits[f32_weights] = dec.forward(x, 0)
            if not f32_weights:
                out = dec.generate(x, N, margins=True)
    for got in logits.values():
        err = float(np.abs(got.astype(np.float64) - ref_logits).max())
        rel = float(np.linalg.norm(got - ref_logits) / np.linalg.norm(ref_logits))
        assert err <= 2e-3 and rel <= 1e-3, (err, rel)
    assert float(np.abs(logits[False].astype(np.float64) - logits[True]).max()) <= 2e-3
    assert greedy.match(out["ids"], ref["ids"], ref["margins"], ref["runner_up"],
                        "bf16-exact weights, 300-position prompt") is None


def test_bf16_prefill_many_prompt_lengths(qa, orc):
    """Every prompt length 65..334: the prefill GEMM's 128-row token tiles end at every possible
    remainder (its rows past the prompt are clamped on load and skipped on store).  Each prefill runs, and
    the last-row logits of lengths 65, 200, 320 and 334 match the oracle's at the prefill tolerance."""
    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=1, bf16=True)
    om = orc.OracleModel.from_product_model(model)
    x_all = qa.prompt_input(model, 324, 10)
    checked = (65, 200, 320, 334)
    with _decoder(qa, model, 340, False) as dec:
        assert dec.weights_bf16
        for T in range(65, 335):
            logits = dec.forward(x_all[:T], 0)
            if T in checked:
                print(f"prefill length {T}", flush=True)
                ref = om.forward_cached(x_all[:T], 0, om.cache(340, True))
                err = float(np.abs(logits.astype(np.float64) - ref).max())
                rel = float(np.linalg.norm(logits - ref) / np.linalg.norm(ref))
                assert err <= 2e-3 and rel <= 1e-3, (T, err, rel)
