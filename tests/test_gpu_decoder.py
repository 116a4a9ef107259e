"""Decoder-level parity: configs 0-4 on the HIP path against the oracle's golden fixtures, greedy
token ids identical, bookkeeping (cur_len, device lengths) bit-exact, reference error behaviour."""
import ctypes
import hashlib
import json
import os
import subprocess

import numpy as np
import pytest
from conftest import LOGIT_ATOL

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()[:16]


def golden(index, bf16=False):
    with open(os.path.join(GOLDEN, f"cfg{index}{'_bf16' if bf16 else ''}.json")) as f:
        return json.load(f)


def close(got, ref, atol=2e-3, rtol_l2=1e-3):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    err = np.abs(got - ref).max()
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err <= atol and rel <= rtol_l2, (err, rel)


@pytest.fixture(scope="module", autouse=True)
def _gpu(qa):
    assert qa.device_count() > 0, "no HIP device: GPU tests need the MI355X"


def test_cfg0_single_layer_decode(qa):
    from qwenasr_amd import configs

    g = golden(0)
    model = qa.Model(configs.CONFIGS[0].size, n_layers=1)
    x, k, v = configs.cfg0_inputs(model.cfg.hidden)
    assert digest(x, k, v, model.tensor("text.blk.0.attn_q.weight")) == g["input_digest"]
    with qa.Decoder(model, 1, 157, qa.QA_CACHE_F32) as dec:
        dec.fill_cache(0, k, v, 156)
        assert dec.cur_len(0) == 156 and dec.device_lens().tolist() == [156]
        y = dec.layer_forward(0, x, 156)
        close(y[0], g["y"], atol=1e-4, rtol_l2=1e-5)
        assert dec.cur_len(0) == g["cur_len"] == 157 and dec.device_lens().tolist() == [157]
        ptr, lay = dec.cache()
        n = lay.n_layers * 2 * lay.n_streams * lay.n_kv_heads * lay.max_seq * lay.head_dim
        cache = np.empty(n, np.float32)
        qa.check(qa.lib.qa_copy_to_host(cache.ctypes.data, ptr, n * 4))
        cache = cache.reshape(1, 2, 1, 8, 157, 128)
        close(cache[0, 0, 0, :, 156], g["k_row"], atol=1e-4, rtol_l2=1e-5)
        close(cache[0, 1, 0, :, 156], g["v_row"], atol=1e-4, rtol_l2=1e-5)
        np.testing.assert_array_equal(cache[0, 0, 0, :, :156], k[0].astype(np.float32))   # prefix untouched


@pytest.mark.parametrize("f16", [True, False])
def test_small_model_greedy_matches_oracle(qa, orc, greedy, f16):
    """0.6B shapes, 3 layers: greedy ids, stop handling and bookkeeping against an in-test oracle run."""
    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=3)
    om = orc.OracleModel.from_product_model(model)
    x = qa.prompt_input(model, 40, 9)
    N = 24
    ref = om.generate(x, N, qa.STOP_IDS, om.cache(49 + N, f16))
    with qa.Decoder(model, 1, 49 + N, qa.QA_CACHE_F16 if f16 else qa.QA_CACHE_F32) as dec:
        out = dec.generate(x, N, margins=True)
        assert greedy.match(out["ids"], ref["ids"], ref["margins"], ref["runner_up"],
                            f"small model ({'f16' if f16 else 'f32'} cache)") is None
        assert out["total_tokens"] == ref["total_tokens"] and out["stopped"] == ref["stopped"]
        assert dec.cur_len(0) == ref["cur_len"] == 49 + N - 1
        assert dec.device_lens().tolist() == [ref["cur_len"]]
        # stop on the 5th generated id: the loop ends right after emitting it (text-decoder.cpp:2282-2292)
        stop = dec.generate(x, N, stop_ids=[ref["ids"][4]])
        first = ref["ids"].index(ref["ids"][4])
        assert stop["stopped"] and stop["ids"] == ref["ids"][:first + 1]
        assert dec.cur_len(0) == 49 + first
        # capacity and argument errors are reported before any device work (text-decoder.cpp:2225-2233)
        with pytest.raises(qa.QaError) as e:
            dec.generate(x, N + 1)
        assert e.value.code == qa.QA_ERR_CAPACITY
        with pytest.raises(qa.QaError) as e:
            dec.forward(x[:2], 49 + N - 1)
        assert e.value.code == qa.QA_ERR_CAPACITY
        # a cached forward of the prompt matches the oracle's logits, to the attention bar of the
        # north star (2e-3 max-abs, 1e-3 relative L2): with an f16 cache, p is rounded to f16, so a
        # 1-ulp f32 difference in a score can move p by one f16 step
        logits = dec.forward(x, 0)
        ref_logits = om.forward_cached(x, 0, om.cache(49 + N, f16))
        close(logits, ref_logits, atol=2e-3, rtol_l2=1e-3)


@pytest.mark.parametrize("persistent", [False, True], ids=["eager", "persistent"])
def test_generate_stop_rolls_back_the_queued_step(qa, persistent):
    """qa_decoder_generate queues the step after id e before it reads id e.  A stop at e undoes that step:
    the length (host and device) counts the fed ids only, and the next call on the same decoder gives what
    a fresh decoder gives.  Stops at the first id (the prefill's pick), at a middle one and at the last."""
    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=2)
    x = qa.prompt_input(model, 20, 6)
    N = 10
    with qa.Decoder(model, 1, 26 + N) as fresh:
        full = fresh.generate(x, N, stop_ids=())
    assert len(full["ids"]) == N and not full["stopped"]
    with qa.Decoder(model, 1, 26 + N) as dec:
        if persistent:
            dec.set_persistent(True)
        for e in (0, 4, N - 1):
            out = dec.generate(x, N, stop_ids=[full["ids"][e]])
            first = full["ids"].index(full["ids"][e])
            assert out["stopped"] and out["ids"] == full["ids"][:first + 1]
            assert out["total_tokens"] == 26 + first + 1
            assert dec.cur_len(0) == 26 + first and dec.device_lens().tolist() == [26 + first]
        again = dec.generate(x, N, stop_ids=())
        assert again["ids"] == full["ids"] and dec.cur_len(0) == 26 + N - 1
        assert dec.device_lens().tolist() == [26 + N - 1]


@pytest.mark.parametrize("index,bf16", [(1, False), (2, False), (3, False), (3, True)])
def test_config_greedy_matches_golden(qa, greedy, index, bf16):
    """Configs 1-3 with seeded N(0, 0.02) f32 weights (the f32 kernels), and config 3 -- the bench
    workload -- with those weights rounded to bf16 values (a converted bf16 checkpoint: the decoder
    streams bf16 copies and the prefill of the 3913-position prompt runs the same kernels)."""
    from qwenasr_amd import configs

    g = golden(index, bf16)
    w = configs.CONFIGS[index]
    model = qa.Model(w.size, n_layers=w.n_layers, bf16=bf16)
    x = qa.prompt_input(model, w.audio_tokens, w.prompt_tokens)
    assert digest(x, model.tensor("text.blk.0.attn_q.weight")) == g["input_digest"]
    label = f"config {index}{' (bf16-exact weights)' if bf16 else ''}"
    print(f"{label}: prompt {w.prompt}, {w.new_tokens} tokens", flush=True)
    with qa.Decoder(model, 1, w.max_seq, w.cache_type) as dec:
        assert dec.weights_bf16 == bf16
        out = dec.generate(x, w.new_tokens, margins=True)
        div = greedy.match(out["ids"], g["ids"], g["margins"], g["runner_up"], label,
                           tie_group="config 3 bf16-exact" if bf16 else None)
        if div is None:
            assert out["stopped"] == g["stopped"] and out["total_tokens"] == g["total_tokens"]
            assert dec.cur_len(0) == g["cur_len"]
        # bookkeeping is exact whatever the ids: one prefill + (n - 1) decode forwards
        assert dec.cur_len(0) == w.prompt + len(out["ids"]) - 1 == out["total_tokens"] - 1
        assert dec.device_lens().tolist() == [dec.cur_len(0)]


@pytest.mark.parametrize("bf16", [False, True])
def test_config4_ragged_streams_match_golden(qa, greedy, bf16):
    """Config 4, all 32 streams, with f32 weights (f32-MFMA skinny GEMMs) and with bf16-exact weights
    (bf16 copies, bf16-MFMA skinny GEMMs over the three-part split of the activations)."""
    from qwenasr_amd import configs

    g = golden(4, bf16)
    w = configs.CONFIGS[4]
    lens = configs.cfg4_lengths(w.streams)
    first = configs.cfg4_first_ids(w.streams)
    assert lens.tolist() == g["lengths"] and first.tolist() == g["first_ids"]
    model = qa.Model(w.size, n_layers=w.n_layers, bf16=bf16)
    with qa.Decoder(model, w.streams, w.max_seq, w.cache_type) as dec:
        assert dec.weights_bf16 == bf16
        for s in range(w.streams):
            k, v = configs.cfg4_stream_kv(s, int(lens[s]))
            dec.fill_cache(s, k, v, int(lens[s]))
            del k, v
        print("config 4 caches filled", flush=True)
        ids = dec.decode_streams(first, w.steps)
        assert ids.shape == (w.steps, w.streams)
        assert sorted(int(s) for s in g["streams"]) == list(range(w.streams))   # every stream has a golden
        for s, ref in g["streams"].items():
            greedy.match(ids[:, int(s)].tolist(), ref["ids"], ref["margins"], ref["runner_up"],
                         f"config 4{' (bf16-exact weights)' if bf16 else ''} stream {s}",
                         tie_group="config 4 bf16-exact" if bf16 else None)
        assert dec.device_lens().tolist() == (lens + w.steps).tolist()
        assert [dec.cur_len(s) for s in range(w.streams)] == (lens + w.steps).tolist()


def _with_env(name, value, fn):
    old = os.environ.get(name)
    os.environ[name] = value
    try:
        return fn()
    finally:
        if old is None:
            os.environ.pop(name, None)
        else:
            os.environ[name] = old


def test_config4_packed_f32_gemms(qa, greedy):
    """QA_GR_PACKED=1 (read at decoder creation): config 4 with the f32 weights on the packed multi-stream GEMMs
    (q|k|v and o on weights reordered for the f32 MFMA, gemm_packed.hip; the LM head is packed by default).  They sum in another order
    than the default kernels, so the comparison runs in its own tie group (at most one accepted near-tie), and the
    bookkeeping stays exact."""
    from qwenasr_amd import configs

    g = golden(4, False)
    w = configs.CONFIGS[4]
    lens = configs.cfg4_lengths(w.streams)
    first = configs.cfg4_first_ids(w.streams)
    model = qa.Model(w.size, n_layers=w.n_layers)
    dec = _with_env("QA_GR_PACKED", "1", lambda: qa.Decoder(model, w.streams, w.max_seq, w.cache_type))
    with dec:
        for s in range(w.streams):
            k, v = configs.cfg4_stream_kv(s, int(lens[s]))
            dec.fill_cache(s, k, v, int(lens[s]))
            del k, v
        print("config 4 (packed f32 GEMMs) caches filled", flush=True)
        ids = dec.decode_streams(first, w.steps)
        for s, ref in g["streams"].items():
            greedy.match(ids[:, int(s)].tolist(), ref["ids"], ref["margins"], ref["runner_up"],
                         f"config 4 (packed f32 GEMMs) stream {s}", tie_group="config 4 packed f32")
        assert dec.device_lens().tolist() == (lens + w.steps).tolist()


@pytest.mark.parametrize("n_streams", [2, 5, 32])
@pytest.mark.parametrize("packed", [False, True])
def test_few_streams_match_oracle(qa, orc, greedy, n_streams, packed):
    """The multi-stream decode step at 2..32 streams (fused RMSNorm / SwiGLU skinny GEMMs, per-stream
    lengths) against the oracle decoding each stream alone: 0.6B shapes, 2 layers, f16 cache, ragged
    contexts, 4 greedy steps; ids identical up to an oracle near-tie."""
    from qwenasr_amd import configs

    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=2)
    om = orc.OracleModel.from_product_model(model)
    rng = np.random.default_rng(n_streams)
    lens = rng.integers(20, 180, n_streams)
    first = rng.integers(0, model.cfg.vocab, n_streams).astype(np.int32)
    steps, cap = 4, 200
    dec = _with_env("QA_GR_PACKED", "1" if packed else "0", lambda: qa.Decoder(model, n_streams, cap, qa.QA_CACHE_F16))
    with dec:
        refs = []
        for s in range(n_streams):
            k, v = configs.cfg4_stream_kv(1000 + s, int(lens[s]), n_layers=2)
            dec.fill_cache(s, k, v, int(lens[s]))
            cache = om.cache(cap, True)
            cache.fill(k, v, int(lens[s]))
            ids, margins, runner = om.decode_steps(cache, int(first[s]), steps)
            refs.append((list(ids), list(margins), list(runner)))
        print(f"{n_streams} streams: oracle done", flush=True)
        got = dec.decode_streams(first, steps)
        for s in range(n_streams):
            greedy.match(got[:, s].tolist(), *refs[s],
                         f"{n_streams}-stream step{' (packed f32 GEMMs)' if packed else ''}, stream {s}")
        assert dec.device_lens().tolist() == (lens + steps).tolist()


def test_decoders_in_sequence_see_cleared_memory(qa):
    """Decoders created one after another in one process, each over memory just released by a buffer
    full of f16 NaN patterns (0xFF bytes), decode identical valid ids: the cache and workspace clears
    complete before the decoder's own (non-blocking) stream runs its first kernel.  Lengths are set
    without filling K/V, so every cache row read is one of the cleared zeros."""
    from qwenasr_amd import configs

    w = configs.CONFIGS[4]
    lens = configs.cfg4_lengths(w.streams)
    first = configs.cfg4_first_ids(w.streams).astype(np.int32)
    model = qa.Model(w.size, n_layers=w.n_layers)
    lay = qa.KvLayout(w.n_layers, w.streams, model.cfg.n_kv_heads, model.cfg.head_dim, w.max_seq, w.cache_type)
    cache_bytes = int(qa.lib.qa_kv_cache_bytes(ctypes.byref(lay)))
    runs = []
    for rep in range(3):
        junk = qa.DeviceArray(cache_bytes, np.uint8, zero=False)
        qa.check(qa.lib.qa_memset_device(junk.ptr, 0xFF, junk.nbytes))
        junk.free()
        with qa.Decoder(model, w.streams, w.max_seq, w.cache_type) as dec:
            for s in range(w.streams):
                dec.set_cur_len(s, int(lens[s]))
            ids = dec.decode_streams(first, 3)
        assert ((ids >= 0) & (ids < model.cfg.vocab)).all(), (rep, ids[:, :8])
        runs.append(ids)
        print(f"decoder {rep}: ids valid", flush=True)
    for ids in runs[1:]:
        np.testing.assert_array_equal(ids, runs[0])


def test_teacher_forced_logits_within_tolerance(qa, orc):
    """Config-4 stream 11 (context 3648, the stream with the smallest oracle margin): GPU and oracle
    decode the same tokens (the oracle's picks) step by step from bit-identical caches; every logit of
    every step agrees to LOGIT_ATOL.  This is the bound the near-tie rule of conftest.GreedyRecorder uses."""
    from qwenasr_amd import configs

    w = configs.CONFIGS[4]
    s = 11
    L = int(configs.cfg4_lengths(w.streams)[s])
    tok = int(configs.cfg4_first_ids(w.streams)[s])
    model = qa.Model(w.size, n_layers=w.n_layers)
    om = orc.OracleModel.from_product_model(model)
    k, v = configs.cfg4_stream_kv(s, L)
    steps = 6
    cache = om.cache(L + steps, True)
    cache.fill(k, v, L)
    worst = 0.0
    with qa.Decoder(model, 1, L + steps, qa.QA_CACHE_F16) as dec:
        dec.fill_cache(0, k, v, L)
        del k, v
        for step in range(steps):
            x = model.embed([tok])
            got = dec.forward(x, L + step)
            ref = om.forward_cached(x, L + step, cache)
            err = float(np.abs(got.astype(np.float64) - ref).max())
            worst = max(worst, err)
            print(f"step {step}: max|dlogit| {err:.2e}", flush=True)
            assert err < LOGIT_ATOL, (step, err)
            tok = int(np.argmax(ref))
    print(f"worst max|dlogit| {worst:.2e} (bound {LOGIT_ATOL})", flush=True)


def test_drop_in_tool_generate(qa, orc):
    """The text-decoder.h drop-in through the synthetic driver, key=value contract, ids vs the oracle."""
    tool = os.path.join(ROOT, "qwenasr.cpp_amd", "qwen-asr-text-layer")
    r = subprocess.run([tool, "--size", "0.6b", "--layers", "2", "--audio-tokens", "20", "--prompt-tokens", "5",
                        "--generate", "6", "--kv-cache-type", "f16", "--device", "gpu"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    kv = dict(line.split("=", 1) for line in r.stdout.strip().splitlines())
    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=2)
    om = orc.OracleModel.from_product_model(model)
    ref = om.generate(qa.prompt_input(model, 20, 5), 6, qa.STOP_IDS, om.cache(31, True))
    assert kv["generated_ids"] == ",".join(map(str, ref["ids"]))
    assert int(kv["prompt_tokens"]) == 25 and int(kv["total_tokens"]) == ref["total_tokens"]
    assert kv["stopped"] == ("true" if ref["stopped"] else "false")
    r = subprocess.run([tool, "--size", "0.6b", "--layers", "1", "--device", "cpu", "--generate", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 1 and "not available" in r.stderr


@pytest.mark.parametrize("bf16", [False, True], ids=["f32-weights", "bf16-copies"])
def test_prefill_is_repeatable(qa, bf16):
    """Three decoders prefill the same 4150-position prompt: the caches and the logits are equal bit for bit.
    The prefill attention splits its last query tiles into two parts over the keys and the part that
    arrives second merges both; the merge rounds every product before the sum, so the result does not
    depend on which part arrives second (with the products fused, the last tiles' rows differed between
    runs, and every later token with them)."""
    m = qa.Model(qa.QWEN3_ASR_1_7B, n_layers=2, bf16=bf16)
    cap, T = 4200, 4150
    x = qa.prompt_input(m, T - 13, 13)
    caches, logits = [], []
    for _ in range(3):
        with qa.Decoder(m, 1, cap, qa.QA_CACHE_F16) as dec:
            logits.append(dec.forward(x, 0))
            ptr, lay = dec.cache()
            n = lay.n_layers * 2 * lay.n_streams * lay.n_kv_heads * lay.max_seq * lay.head_dim
            c = np.empty(n, np.float16)
            qa.check(qa.lib.qa_copy_to_host(c.ctypes.data, ptr, n * 2))
            caches.append(c.reshape(2, 2, 8, cap, 128)[:, :, :, :T])
    for r in (1, 2):
        np.testing.assert_array_equal(caches[r], caches[0])
        np.testing.assert_array_equal(logits[r], logits[0])
