"""Pins the CPU oracle (oracle/qa_oracle.c) before it is trusted as the checker of the HIP path.

The reference holds no golden vectors for synthetic inputs (its parity scripts need a real HF
checkpoint and a WAV), so each oracle function is checked against something that fixes it
independently: a library routine (numpy float16 casts, torch scaled_dot_product_attention, float64
matmul), a closed form written from the mathematics, or an invariant that a plausible mistake breaks
(interleaved instead of NEOX pairs, a missing eps, a wrong GQA mapping, a dropped residual, an
off-by-one position).
"""
import math
import os

import numpy as np
import pytest


class _LazyTorch:
    """torch, imported on first use: only these CPU cross-checks need it, and a GPU session that
    collects this file must not load torch's own HIP runtime next to the library's."""

    def __getattr__(self, name):
        import torch as _torch

        return getattr(_torch, name)


torch = _LazyTorch()


# ---------------------------------------------------------------------------------------------- f16
def test_f32_to_f16_matches_numpy_rne(orc):
    rng = np.random.default_rng(0)
    vals = [rng.standard_normal(20000).astype(np.float32) * np.float32(s) for s in (1e-8, 1e-6, 1e-4, 1e-2, 1, 1e2, 1e4)]
    special = np.array([0.0, -0.0, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 65504.0, 65519.99, 65520.0, 70000.0,
                        -65520.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14 - 2.0 ** -25, 1e-30,
                        np.inf, -np.inf, np.nan], dtype=np.float32)
    x = np.concatenate(vals + [special])
    ours = orc.f32_to_f16_bits(x)
    ref = x.astype(np.float16).view(np.uint16)
    finite = ~np.isnan(x)
    np.testing.assert_array_equal(ours[finite], ref[finite])
    assert np.isnan(orc.f16_bits_to_f32(ours[~finite])).all()
    # and back: f16 -> f32 is exact for every bit pattern
    allbits = np.arange(65536, dtype=np.uint16)
    back = orc.f16_bits_to_f32(allbits)
    ref_back = allbits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref_back)
    np.testing.assert_array_equal(back[~nan].view(np.uint32), ref_back[~nan].view(np.uint32))


# ---------------------------------------------------------------------------------------------- RMSNorm
def test_rms_norm_closed_form(orc):
    rng = np.random.default_rng(1)
    for n in (128, 1024, 2048):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        eps = 1e-6
        y = orc.rms_norm_row(x, w, eps)
        xd = x.astype(np.float64)
        ref = xd / np.sqrt(np.mean(xd * xd) + eps) * w
        np.testing.assert_allclose(y, ref, rtol=3e-7, atol=0)
    # eps matters for tiny inputs: a dropped eps would blow this up
    x = np.full(128, 1e-5, dtype=np.float32)
    y = orc.rms_norm_row(x, np.ones(128, np.float32), 1e-6)
    np.testing.assert_allclose(y, 1e-5 / math.sqrt(1e-10 + 1e-6), rtol=1e-6)


# ---------------------------------------------------------------------------------------------- RoPE
def _rope_closed_form(rows: np.ndarray, pos: int, theta: float) -> np.ndarray:
    d = rows.shape[-1]
    half = d // 2
    i = np.arange(half, dtype=np.float64)
    ang = pos * theta ** (-2.0 * i / d)
    c, s = np.cos(ang), np.sin(ang)
    a, b = rows[:, :half].astype(np.float64), rows[:, half:].astype(np.float64)
    return np.concatenate([a * c - b * s, b * c + a * s], axis=1)


def test_rope_neox_closed_form(orc):
    rng = np.random.default_rng(2)
    rows = rng.standard_normal((8, 128)).astype(np.float32)
    for pos in (0, 1, 7, 156, 3913, 4168):
        got = orc.rope_rows(rows, pos, 1.0e6)
        np.testing.assert_allclose(got, _rope_closed_form(rows, pos, 1.0e6), rtol=2e-6, atol=2e-6)
    np.testing.assert_array_equal(orc.rope_rows(rows, 0, 1.0e6), rows)          # position 0 is identity
    got = orc.rope_rows(rows, 1234, 1.0e6)                                       # pair norms preserved
    np.testing.assert_allclose(got[:, :64] ** 2 + got[:, 64:] ** 2, rows[:, :64] ** 2 + rows[:, 64:] ** 2, rtol=1e-5)
    # an interleaved (GPT-J) pairing (2i, 2i + 1) is a different rotation: the oracle must not match it
    ang = 156 * 1.0e6 ** (-2.0 * np.arange(64) / 128)
    a, b = rows[:, 0::2].astype(np.float64), rows[:, 1::2].astype(np.float64)
    gptj = np.empty((8, 128))
    gptj[:, 0::2] = a * np.cos(ang) - b * np.sin(ang)
    gptj[:, 1::2] = b * np.cos(ang) + a * np.sin(ang)
    assert not np.allclose(orc.rope_rows(rows, 156, 1.0e6), gptj, atol=1e-3)


def test_rope_matches_hf_rotate_half_formula(orc):
    # the reference's Torch check (benchmarks/check_text_layer0.py:98-110) uses cat(freqs, freqs) and rotate_half
    rng = np.random.default_rng(3)
    q = torch.from_numpy(rng.standard_normal((5, 16, 128)).astype(np.float64))
    pos = torch.arange(5, dtype=torch.float64) + 150
    inv = 1.0 / (1.0e6 ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128))
    emb = torch.cat([torch.outer(pos, inv)] * 2, dim=-1)
    rot = torch.cat([-q[..., 64:], q[..., :64]], dim=-1)
    ref = q * emb.cos()[:, None] + rot * emb.sin()[:, None]
    for t in range(5):
        got = orc.rope_rows(q[t].numpy().astype(np.float32), 150 + t, 1.0e6)
        np.testing.assert_allclose(got, ref[t].numpy(), rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------------------------------------- linear
def test_linear_matches_float64_and_is_batch_independent(orc):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((7, 1024)).astype(np.float32)
    w = (rng.standard_normal((301, 1024)) * 0.02).astype(np.float32)
    y = orc.linear(x, w)
    np.testing.assert_allclose(y, x.astype(np.float64) @ w.astype(np.float64).T, rtol=1e-4, atol=2e-5)
    for r in range(7):  # a row's result never depends on the other rows of the batch
        np.testing.assert_array_equal(orc.linear(x[r:r + 1], w)[0], y[r])


# ---------------------------------------------------------------------------------------------- argmax
def test_argmax_first_max_nan_and_empty(orc):
    assert orc.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert orc.argmax(np.array([np.nan, 0.5, np.nan, 0.5], np.float32)) == 1
    assert orc.argmax(np.array([-np.inf, -np.inf], np.float32)) == -1
    assert orc.argmax(np.array([np.nan, np.nan], np.float32)) == -1
    assert orc.argmax(np.array([-np.inf, -1e38], np.float32)) == 1


# ---------------------------------------------------------------------------------------------- attention
def _sdpa(q, k, v, n_past, causal_rows=True):
    """float64 torch SDPA with GQA h -> h // 2 and the cached causal limit key <= n_past + t."""
    T, H, d = q.shape
    n_kv, L, _ = k.shape
    rep = H // n_kv
    qt = torch.from_numpy(q.astype(np.float64)).permute(1, 0, 2)                  # [H][T][d]
    kt = torch.from_numpy(k.astype(np.float64)).repeat_interleave(rep, dim=0)     # [H][L][d]
    vt = torch.from_numpy(v.astype(np.float64)).repeat_interleave(rep, dim=0)
    mask = torch.arange(L)[None, :] <= (n_past + torch.arange(T))[:, None]
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask)
    return out.permute(1, 0, 2).numpy()


@pytest.mark.parametrize("n_past,T", [(0, 1), (5, 1), (156, 1), (0, 37), (20, 13)])
def test_cache_attention_f32_matches_sdpa(orc, n_past, T):
    rng = np.random.default_rng(5 + n_past + T)
    L = n_past + T
    q = rng.standard_normal((T, 16, 128)).astype(np.float32)
    k = rng.standard_normal((8, L, 128)).astype(np.float32)
    v = rng.standard_normal((8, L, 128)).astype(np.float32)
    got = orc.cache_attention(k, v, q, n_past, f16=False)
    np.testing.assert_allclose(got, _sdpa(q, k, v, n_past), rtol=1e-5, atol=2e-6)


def test_cache_attention_f16_semantics(orc):
    """f16 cache: within the path tolerance of the exact result on f16-stored K/V, and the q/p rounding
    points of GGML's f16 mul_mat are really applied (result differs from plain f32 arithmetic)."""
    rng = np.random.default_rng(6)
    n_past, T = 300, 3
    L = n_past + T
    q = rng.standard_normal((T, 16, 128)).astype(np.float32)
    k = rng.standard_normal((8, L, 128)).astype(np.float32)
    v = rng.standard_normal((8, L, 128)).astype(np.float32)
    k16 = k.astype(np.float16).astype(np.float32)
    v16 = v.astype(np.float16).astype(np.float32)
    got = orc.cache_attention(k, v, q, n_past, f16=True)
    exact = _sdpa(q, k16, v16, n_past)
    assert np.abs(got - exact).max() <= 2e-3
    assert np.linalg.norm(got - exact) / np.linalg.norm(exact) <= 1e-3
    plain = orc.cache_attention(k16, v16, q, n_past, f16=False)
    assert np.abs(got - plain).max() > 0   # q -> f16 and p -> f16 change the result


# The f16-cache attention semantics, pinned at their rounding points.  GGML's f16 mul_mat converts
# src1 to f16 (q before QK^T, p before PV) and soft_max_ext normalises in f32 before that conversion
# (text-decoder.cpp:454-461 [ggml-sem]).  The inputs below make every q.K dot product exact in f32, so
# a float64 statement with f32 rounding applied exactly where those ops round matches the oracle to
# f32 accumulation error, and misplaced roundings are far outside that bar.
PIN_REL = 1e-6


def _exact_f16_values(rng, shape):
    """a * 2^-4 with integer |a| in [1, 64]: exact in f16; a product of two is a multiple of 2^-8 below 16,
    so any 128-term dot product of them is exact in f32, in any summation order."""
    a = rng.integers(1, 65, shape) * rng.choice([-1, 1], shape)
    return (a * 2.0 ** -4).astype(np.float32)


def _f16_attention_statement(q, k16, v16, n_past, round_q=True, p_round="normalised"):
    """float64 statement: q -> f16; s = f32(f32(q16 . K16) * f32(1/sqrt(d))); M = max s;
    e = f32(exp(s - M)); S = double sum of e; p = f16(f32(e * f32(1/S))); o = sum_j p_j V16_j.
    round_q=False and p_round="unnormalised" (p = f16(e) * f32(1/S)) state the two misplaced roundings."""
    T, H, d = q.shape
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    qq = q.astype(np.float16).astype(np.float64) if round_q else q.astype(np.float64)
    out = np.zeros((T, H, d))
    for t in range(T):
        n = n_past + t + 1
        for h in range(H):
            K, V = k16[h // 2, :n].astype(np.float64), v16[h // 2, :n].astype(np.float64)
            s = (K @ qq[t, h]).astype(np.float32) * scale
            e = np.exp((s - s.max()).astype(np.float64)).astype(np.float32)
            r = np.float32(1.0 / float(np.sum(e.astype(np.float64))))
            if p_round == "normalised":
                p = (e * r).astype(np.float16)
            else:
                p = e.astype(np.float16).astype(np.float32) * r
            out[t, h] = p.astype(np.float64) @ V
    return out


def _pin_inputs(n_past, T, seed):
    rng = np.random.default_rng(seed)
    L = n_past + T
    q16 = _exact_f16_values(rng, (T, 16, 128))
    # q carries bits below half an f16 ulp of q16: rounding q to f16 gives q16 back
    ulp = 2.0 ** (np.floor(np.log2(np.abs(q16))) - 11)   # the smaller of the ulps either side of q16
    q = (q16 + 0.45 * ulp * rng.uniform(-1, 1, q16.shape)).astype(np.float32)
    assert (q.astype(np.float16).astype(np.float32) == q16).all()
    k = _exact_f16_values(rng, (8, L, 128))
    v = rng.standard_normal((8, L, 128)).astype(np.float32)
    return q, k, v.astype(np.float16).astype(np.float32)


def _rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("n_past,T", [(0, 1), (157, 1), (300, 3), (1000, 1)])
def test_cache_attention_f16_rounding_points_pinned(orc, n_past, T):
    q, k, v16 = _pin_inputs(n_past, T, 60 + n_past + T)
    got = orc.cache_attention(k, v16, q, n_past, f16=True)
    want = _f16_attention_statement(q, k, v16, n_past)
    assert _rel(got, want) <= PIN_REL, _rel(got, want)
    # the misplaced roundings are far outside the bar: the pin tells them apart from the oracle
    if n_past > 0:
        for kw in (dict(round_q=False), dict(p_round="unnormalised")):
            assert _rel(_f16_attention_statement(q, k, v16, n_past, **kw), want) > 20 * PIN_REL, kw


@pytest.fixture(scope="module")
def planted_builds(tmp_path_factory, orc):
    """Copies of the oracle built with a planted mistake (ORC_PLANT in qa_oracle.c): 1 rounds p before the
    normalisation, 2 leaves q unrounded."""
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("gcc is needed to build the planted-mistake oracles")
    out = {}
    src = os.path.join(orc.ORACLE_DIR, "qa_oracle.c")
    for plant in (1, 2):
        so = str(tmp_path_factory.mktemp(f"plant{plant}") / "libqa_oracle_plant.so")
        subprocess.run(["gcc", "-O3", "-std=c11", "-fPIC", "-fopenmp", "-ffp-contract=off", "-march=x86-64-v3",
                        f"-DORC_PLANT={plant}", "-shared", "-o", so, src, "-lm"], check=True, capture_output=True)
        out[plant] = orc.load_build(so)
    return out


@pytest.mark.parametrize("plant", [1, 2])
def test_attention_pin_rejects_planted_mistakes(orc, planted_builds, plant):
    """Negative controls: an oracle with p rounded before the normalisation (1) or q left unrounded (2)
    fails the pin above, and matches the statement of its own mistake instead."""
    n_past, T = 300, 3
    q, k, v16 = _pin_inputs(n_past, T, 60 + n_past + T)
    bad = orc.cache_attention(k, v16, q, n_past, f16=True, library=planted_builds[plant])
    want = _f16_attention_statement(q, k, v16, n_past)
    assert _rel(bad, want) > 20 * PIN_REL, _rel(bad, want)
    if plant == 1:
        assert _rel(bad, _f16_attention_statement(q, k, v16, n_past, p_round="unnormalised")) <= PIN_REL


def test_attention_special_cases(orc):
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, 16, 128)).astype(np.float32)
    k = rng.standard_normal((8, 1, 128)).astype(np.float32)
    v = rng.standard_normal((8, 1, 128)).astype(np.float32)
    for f16 in (False, True):                       # L = 1 -> o = V_0 (p = 1 exactly, also in f16)
        got = orc.cache_attention(k, v, q, 0, f16)
        vv = v.astype(np.float16).astype(np.float32) if f16 else v
        np.testing.assert_array_equal(got, np.repeat(vv[:, 0], 2, axis=0)[None])
    L = 50                                          # identical keys -> mean of V
    k = np.repeat(rng.standard_normal((8, 1, 128)).astype(np.float32), L, axis=1)
    v = rng.standard_normal((8, L, 128)).astype(np.float32)
    got = orc.cache_attention(k, v, rng.standard_normal((1, 16, 128)).astype(np.float32), L - 1, False)
    np.testing.assert_allclose(got[0], np.repeat(v.mean(axis=1), 2, axis=0), rtol=1e-5, atol=1e-6)
    k = np.zeros((8, L, 128), np.float32)           # one dominant score -> that V row
    qd = np.zeros((1, 16, 128), np.float32)
    k[:, 17, 0] = 100.0
    qd[0, :, 0] = 100.0
    got = orc.cache_attention(k, v, qd, L - 1, False)
    np.testing.assert_allclose(got[0], np.repeat(v[:, 17], 2, axis=0), atol=1e-6)


def test_gqa_maps_head_h_to_kv_head_h_div_2(orc):
    rng = np.random.default_rng(8)
    L = 40
    q = rng.standard_normal((1, 16, 128)).astype(np.float32)
    k = rng.standard_normal((8, L, 128)).astype(np.float32)
    v = rng.standard_normal((8, L, 128)).astype(np.float32)
    got = orc.cache_attention(k, v, q, L - 1, False)[0]
    for h in range(16):
        one = orc.cache_attention(k[h // 2:h // 2 + 1], v[h // 2:h // 2 + 1], q[:, h:h + 1], L - 1, False)[0, 0]
        np.testing.assert_array_equal(got[h], one)
    wrong = orc.cache_attention(k[3:4], v[3:4], q[:, 1:2], L - 1, False)[0, 0]   # h % 8 mapping for h = 11
    assert not np.allclose(got[11], wrong)


def test_causal_f32_matches_sdpa(orc):
    rng = np.random.default_rng(9)
    T = 45
    q = rng.standard_normal((T, 16, 128)).astype(np.float32)
    k = rng.standard_normal((T, 8, 128)).astype(np.float32)
    v = rng.standard_normal((T, 8, 128)).astype(np.float32)
    got = orc.causal_attention_f32(q, k, v)
    ref = _sdpa(q, k.transpose(1, 0, 2), v.transpose(1, 0, 2), 0)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=2e-6)


# ---------------------------------------------------------------------------------------------- layers
def _tiny_cfg(layers=2, hidden=256, inter=512, vocab=97):
    return dict(n_layers=layers, hidden=hidden, n_heads=16, n_kv_heads=8, head_dim=128, intermediate=inter,
                vocab=vocab, rope_theta=1.0e6, rms_norm_eps=1e-6)


def _tiny_model(orc, cfg, seed=11):
    rng = np.random.default_rng(seed)
    H, QD, KD, I = cfg["hidden"], 16 * 128, 8 * 128, cfg["intermediate"]

    def n(*shape, s=0.02):
        return (rng.standard_normal(shape) * s).astype(np.float32)

    layers = []
    for _ in range(cfg["n_layers"]):
        layers.append(dict(attn_norm=1 + n(H, s=0.1), ffn_norm=1 + n(H, s=0.1), q=n(QD, H), k=n(KD, H), v=n(KD, H),
                           o=n(H, QD), q_norm=1 + n(128, s=0.1), k_norm=1 + n(128, s=0.1), gate=n(I, H), up=n(I, H),
                           down=n(H, I)))
    embd = n(cfg["vocab"], H, s=1.0)
    out_norm = 1 + n(H, s=0.1)
    model = orc.OracleModel(cfg, layers, embd, out_norm, embd)
    model.output_norm_w = out_norm
    return model, layers, embd


def _torch_layer(x, lw, cfg, pos0=0):
    """Qwen3 decoder layer from its definition (float64, causal, positions pos0..)."""
    d = torch.float64
    X = torch.from_numpy(x).to(d)
    t = {k: torch.from_numpy(v).to(d) for k, v in lw.items()}

    def rms(a, w):
        return a / torch.sqrt(a.pow(2).mean(-1, keepdim=True) + cfg["rms_norm_eps"]) * w

    T = X.shape[0]
    hcur = rms(X, t["attn_norm"])
    q = (hcur @ t["q"].T).view(T, 16, 128)
    k = (hcur @ t["k"].T).view(T, 8, 128)
    v = (hcur @ t["v"].T).view(T, 8, 128)
    q, k = rms(q, t["q_norm"]), rms(k, t["k_norm"])
    pos = torch.arange(T, dtype=d) + pos0
    inv = cfg["rope_theta"] ** (-torch.arange(0, 128, 2, dtype=d) / 128)
    ang = torch.outer(pos, inv)
    c, s = ang.cos()[:, None], ang.sin()[:, None]

    def rope(a):
        a1, a2 = a[..., :64], a[..., 64:]
        return torch.cat([a1 * c - a2 * s, a2 * c + a1 * s], dim=-1)

    q, k = rope(q), rope(k)
    kk, vv = k.repeat_interleave(2, dim=1), v.repeat_interleave(2, dim=1)
    att = torch.nn.functional.scaled_dot_product_attention(q.permute(1, 0, 2), kk.permute(1, 0, 2),
                                                           vv.permute(1, 0, 2), is_causal=True)
    att = att.permute(1, 0, 2).reshape(T, 16 * 128)
    X = X + att @ t["o"].T
    hcur = rms(X, t["ffn_norm"])
    g, u = hcur @ t["gate"].T, hcur @ t["up"].T
    X = X + (torch.nn.functional.silu(g) * u) @ t["down"].T
    return X.numpy()


def test_layer_nocache_matches_textbook_qwen3_layer(orc):
    cfg = _tiny_cfg(layers=1)
    m, layers, _ = _tiny_model(orc, cfg)
    x = np.random.default_rng(12).standard_normal((20, cfg["hidden"])).astype(np.float32)
    got = m.layer_forward_nocache(0, x)
    np.testing.assert_allclose(got, _torch_layer(x, layers[0], cfg), rtol=1e-4, atol=2e-5)


def test_layer_cached_prefix_then_decode_matches_full_sequence(orc):
    """Cache write at n_past, positions n_past + t and attend-after-append, against the full causal layer."""
    cfg = _tiny_cfg(layers=1)
    m, layers, _ = _tiny_model(orc, cfg)
    x = np.random.default_rng(13).standard_normal((12, cfg["hidden"])).astype(np.float32)
    full = _torch_layer(x, layers[0], cfg)
    cache = m.cache(16, f16=False)
    y0 = m.layer_forward_cached(0, x[:9], 0, cache)
    y1 = m.layer_forward_cached(0, x[9:10], 9, cache)
    y2 = m.layer_forward_cached(0, x[10:12], 10, cache)
    np.testing.assert_allclose(np.concatenate([y0, y1, y2]), full, rtol=1e-4, atol=2e-5)
    assert cache.cur_len == 12
    assert not cache.k[0, :, 12:].any() and not cache.v[0, :, 12:].any()     # rows past cur_len untouched
    # the f32 cached path and the non-cached path are the same arithmetic
    np.testing.assert_array_equal(y0, m.layer_forward_nocache(0, x[:9]))


def test_generate_cached_equals_recompute_greedy(orc):
    """qwenasr_text_generate_cached_* and qwenasr_text_generate_greedy_cpu produce the same ids
    (text-decoder.cpp:1920-2016 vs 2033-2207); 1 prefill + (N - 1) decode forwards."""
    cfg = _tiny_cfg(layers=2)
    m, _, embd = _tiny_model(orc, cfg)
    x = np.random.default_rng(14).standard_normal((6, cfg["hidden"])).astype(np.float32)
    N = 7
    cache = m.cache(6 + N, f16=False)
    out = m.generate(x, N, [], cache)
    assert out["rc"] == 0 and len(out["ids"]) == N and not out["stopped"]
    assert out["total_tokens"] == 6 + N and out["cur_len"] == 6 + N - 1
    seq = x
    ids = []
    for _ in range(N):
        nid = orc.argmax(m.prefill_nocache(seq))
        ids.append(nid)
        seq = np.concatenate([seq, embd[nid:nid + 1]])
    assert ids == out["ids"]
    # stop id: generation ends right after emitting it
    stop = m.generate(x, N, [out["ids"][2]], m.cache(6 + N, f16=False))
    first = out["ids"].index(out["ids"][2])
    assert stop["stopped"] and stop["ids"] == out["ids"][:first + 1] and stop["total_tokens"] == 6 + first + 1
    assert m.generate(x, 0, [], m.cache(6, f16=False))["ids"] == []
    assert m.generate(x, N, [], m.cache(6 + N - 1, f16=False))["rc"] == 2      # exceeds KV-cache capacity


def test_decode_steps_continue_generate(orc):
    """orc_decode_steps (the per-stream statement of config 4) continued from the cache a prefill left
    gives exactly what orc_generate_cached gives after its first pick: same ids, margins, runner-ups and
    cur_len (1 prefill + N - 1 decode forwards, text-decoder.cpp:2209-2311)."""
    cfg = _tiny_cfg(layers=2)
    m, _, _ = _tiny_model(orc, cfg)
    x = np.random.default_rng(16).standard_normal((6, cfg["hidden"])).astype(np.float32)
    N = 7
    for f16 in (False, True):
        gen = m.generate(x, N, [], m.cache(6 + N, f16))
        cache = m.cache(6 + N, f16)
        m.forward_cached(x, 0, cache)
        assert cache.cur_len == 6
        ids, marg, second = m.decode_steps(cache, gen["ids"][0], N - 1)
        assert ids == gen["ids"][1:] and marg == gen["margins"][1:] and second == gen["runner_up"][1:], f16
        assert cache.cur_len == gen["cur_len"] == 6 + N - 1


def _torch_decode(layers, embd, out_norm, cfg, k0, v0, first, n_steps):
    """Greedy decode from token `first` over a cache pre-filled with rows k0, v0 [layer][kv head][L0][d]
    (K held after k_norm and RoPE, as the reference stores it), Qwen3 layers from their definition in
    float64: step i embeds the token, appends its k/v at position L0 + i and attends over 0..L0 + i."""
    d = torch.float64
    eps = cfg["rms_norm_eps"]
    W = [{k: torch.from_numpy(v).to(d) for k, v in lw.items()} for lw in layers]
    E, ON = torch.from_numpy(embd).to(d), torch.from_numpy(out_norm).to(d)
    Kc = [torch.from_numpy(k0[l]).to(d) for l in range(len(layers))]
    Vc = [torch.from_numpy(v0[l]).to(d) for l in range(len(layers))]
    inv = cfg["rope_theta"] ** (-torch.arange(0, 128, 2, dtype=d) / 128)

    def rms(a, w):
        return a / torch.sqrt(a.pow(2).mean(-1, keepdim=True) + eps) * w

    tok, ids, margins = first, [], []
    L0 = k0.shape[2]
    for step in range(n_steps):
        ang = (L0 + step) * inv
        c, s = ang.cos(), ang.sin()

        def rope(a):
            return torch.cat([a[..., :64] * c - a[..., 64:] * s, a[..., 64:] * c + a[..., :64] * s], dim=-1)

        X = E[tok][None]
        for l, w in enumerate(W):
            h = rms(X, w["attn_norm"])
            q = rope(rms((h @ w["q"].T).view(16, 128), w["q_norm"]))
            k = rope(rms((h @ w["k"].T).view(8, 128), w["k_norm"]))
            v = (h @ w["v"].T).view(8, 128)
            Kc[l] = torch.cat([Kc[l], k[:, None]], dim=1)
            Vc[l] = torch.cat([Vc[l], v[:, None]], dim=1)
            Kh, Vh = Kc[l].repeat_interleave(2, dim=0), Vc[l].repeat_interleave(2, dim=0)
            p = torch.softmax((Kh @ q[:, :, None])[..., 0] / math.sqrt(128), dim=-1)
            att = (p[:, None, :] @ Vh)[:, 0]
            X = X + att.reshape(1, -1) @ w["o"].T
            h = rms(X, w["ffn_norm"])
            X = X + (torch.nn.functional.silu(h @ w["gate"].T) * (h @ w["up"].T)) @ w["down"].T
        logits = (rms(X, ON) @ E.T)[0]
        top = torch.topk(logits, 2)
        tok = int(top.indices[0])
        ids.append(tok)
        margins.append(float(top.values[0] - top.values[1]))
    return ids, margins, [k.numpy() for k in Kc], [v.numpy() for v in Vc]


def test_decode_steps_match_textbook_decode_over_prefilled_cache(orc):
    """orc_decode_steps from a cache pre-filled with random rows (config 4's setting) against the float64
    textbook decode: identical greedy ids (every float64 top-2 margin here is far above f32 error), the
    appended K/V rows at positions L0.., and cur_len = L0 + steps."""
    cfg = _tiny_cfg(layers=2)
    m, layers, embd = _tiny_model(orc, cfg)
    rng = np.random.default_rng(17)
    L0, steps = 40, 6
    k0 = rng.standard_normal((2, 8, L0, 128)).astype(np.float32)
    v0 = rng.standard_normal((2, 8, L0, 128)).astype(np.float32)
    ids_ref, marg_ref, K, V = _torch_decode(layers, embd, m.output_norm_w, cfg, k0, v0, 5, steps)
    assert min(marg_ref) > 1e-3, marg_ref
    cache = m.cache(L0 + steps, f16=False)
    cache.fill(k0, v0, L0)
    ids, marg, _ = m.decode_steps(cache, 5, steps)
    assert ids == ids_ref
    np.testing.assert_allclose(marg, marg_ref, rtol=1e-3, atol=1e-4)
    assert cache.cur_len == L0 + steps
    np.testing.assert_allclose(cache.k[:, :, L0:L0 + steps], np.stack(K)[:, :, L0:L0 + steps], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(cache.v[:, :, L0:L0 + steps], np.stack(V)[:, :, L0:L0 + steps], rtol=1e-4, atol=1e-5)
    np.testing.assert_array_equal(cache.k[:, :, :L0], k0)          # the prefilled rows are never rewritten


# ---------------------------------------------------------------------------------------------- bookkeeping
def test_slot_index_positions_mask(orc, qa):
    import ctypes

    lay = qa.KvLayout(1, 1, 8, 128, 220, qa.QA_CACHE_F16)
    rng = np.random.default_rng(15)
    for _ in range(200):
        h, p, i = int(rng.integers(8)), int(rng.integers(220)), int(rng.integers(128))
        ref = (h * 220 + p) * 128 + i                      # ne = [128, max_seq, 8] (text-decoder.cpp:1451-1462)
        assert orc.lib.orc_slot_index(h, p, i, 220, 128) == ref
        assert qa.lib.qa_kv_slot_index(ctypes.byref(lay), 0, 0, 0, h, p, i) == ref
    pos = np.zeros(13, np.int32)
    qa.check(qa.lib.qa_positions(156, 13, qa.iptr(pos)))
    np.testing.assert_array_equal(pos, np.arange(156, 169))
    for n_past, T in ((0, 5), (7, 3), (156, 1)):
        mq = np.zeros(T * (n_past + T), np.float32)
        mo = np.zeros(T * (n_past + T), np.float32)
        qa.check(qa.lib.qa_causal_mask(n_past, T, qa.fptr(mq)))
        orc.lib.orc_causal_mask(n_past, T, orc.fptr(mo))
        np.testing.assert_array_equal(mq.view(np.uint32), mo.view(np.uint32))
        ref = np.where(np.arange(n_past + T)[None, :] <= n_past + np.arange(T)[:, None], 0.0, -np.inf)
        np.testing.assert_array_equal(mq.reshape(T, -1), ref.astype(np.float32))
