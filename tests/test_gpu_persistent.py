"""GPU tests of the persistent decode step (qa_decoder_set_persistent).

Each batch-1 decode step of a persistent decoder runs every layer in one launch whose phases
call the same device functions as the eager launches, so the ids, logits and lengths must equal the
eager decoder's bit for bit.  The eager step is held to the oracle by the other GPU tests; the short
cases here also compare the ids with the oracle directly.  Every call goes through the C ABI.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu(qa):
    assert qa.device_count() > 0, "no HIP device: GPU tests need the MI355X"


def decode(qa, model, cap, cache, x, n_new, persistent):
    """Greedy generation, then a teacher-forced cached forward of one token after the prompt."""
    with qa.Decoder(model, 1, cap, cache) as d:
        if persistent:
            d.set_persistent(True)
        g = d.generate(x, n_new)
        lens = d.device_lens().tolist()
        cur = d.cur_len(0)
        n = x.shape[0]
        logits = d.forward(model.embed([g["ids"][0]]), n)
        return g["ids"], logits, lens, cur, d.device_lens().tolist()


@pytest.mark.parametrize("size", ["0.6B", "1.7B"])
@pytest.mark.parametrize("cache", ["f16", "f32"])
@pytest.mark.parametrize("bf16", [False, True], ids=["f32-weights", "bf16-copies"])
def test_persistent_step_bit_identical_short_cache(qa, orc, size, cache, bf16):
    """A 36-position cache (scores and values chunks of 32): both model shapes, both cache dtypes, f32
    weights and the bf16 copies of bf16-exact weights."""
    shape = qa.QWEN3_ASR_0_6B if size == "0.6B" else qa.QWEN3_ASR_1_7B
    ct = qa.QA_CACHE_F16 if cache == "f16" else qa.QA_CACHE_F32
    m = qa.Model(shape, n_layers=2, bf16=bf16)
    x = qa.prompt_input(m, 24, 6)
    eager = decode(qa, m, 36, ct, x, 6, False)
    pers = decode(qa, m, 36, ct, x, 6, True)
    assert pers[0] == eager[0]
    np.testing.assert_array_equal(pers[1], eager[1])
    assert pers[2] == eager[2] == [35] and pers[3] == eager[3] == 35
    assert pers[4] == eager[4] == [31]
    om = orc.OracleModel.from_product_model(m)
    ref = om.generate(x, 6, qa.STOP_IDS, om.cache(36, ct == qa.QA_CACHE_F16))
    assert pers[0] == ref["ids"]


# (capacity, prompt): one capacity per batch-1 tiling the decoder can pick for each cache dtype (scores chunk /
# values chunk / statistics register slots / merge loads); the 36-position cache of the test above takes
# 32 / 32 / 1 / 8
LONG_F16 = [(600, 560, "32-64"), (1500, 1450, "64-128"), (2600, 2560, "128-128-mb16"), (4200, 4150, "144-256"),
            (4800, 4750, "160-256"), (5500, 5450, "192-256"), (7000, 6950, "128-256-mb16"), (9000, 8950, "128-256-sr2"),
            (17000, 16950, "128-256-sr4"), (33000, 32950, "128-256-sr8")]
LONG_F32 = [(900, 860, "32-32-mb16"), (1200, 1150, "32-64"), (1800, 1750, "64-64"), (2300, 2250, "64-128"),
            (3000, 2950, "128-128"), (5000, 4950, "160-256")]
LONG = [(cap, prompt, f"f16-{t}", "f16") for cap, prompt, t in LONG_F16] + \
       [(cap, prompt, f"f32-{t}", "f32") for cap, prompt, t in LONG_F32]


@pytest.mark.parametrize("cap, prompt, tiling, cache", LONG, ids=[t for _, _, t, _ in LONG])
def test_persistent_step_bit_identical_long_cache(qa, cap, prompt, tiling, cache):
    """The tilings of longer caches: several scores blocks and values merge participants per KV head, so the
    values phase's merge runs (1.7B shape, 2 layers)."""
    m = qa.Model(qa.QWEN3_ASR_1_7B, n_layers=2)
    ct = qa.QA_CACHE_F16 if cache == "f16" else qa.QA_CACHE_F32
    x = qa.prompt_input(m, prompt - 13, 13)
    print(f"persistent long cache {tiling}: capacity {cap}, prompt {prompt}", flush=True)
    eager = decode(qa, m, cap, ct, x, 8, False)
    pers = decode(qa, m, cap, ct, x, 8, True)
    assert pers[0] == eager[0]
    np.testing.assert_array_equal(pers[1], eager[1])
    assert pers[2:] == eager[2:]


# every capacity at which the batch-1 tiling changes, and the largest covered
EDGES = [1, 512, 513, 1024, 1025, 1280, 1281, 2048, 2049, 2560, 2561, 4096, 4097, 4608, 4609, 5120, 5121, 6144, 6145,
         8192, 8193, 16384, 16385, 32768, 32769, 65536]


@pytest.mark.parametrize("size", ["0.6B", "1.7B"])
@pytest.mark.parametrize("cache", ["f16", "f32"])
def test_persistent_step_covers_every_capacity(qa, size, cache):
    """Both model shapes and cache dtypes have a persistent kernel for every tiling, at the capacities where
    the tiling changes (small vocabulary: only the layer kernels matter here)."""
    base = qa.QWEN3_ASR_0_6B if size == "0.6B" else qa.QWEN3_ASR_1_7B
    shape = qa.ModelSize(base.name + "-v4096", hidden=base.hidden, intermediate=base.intermediate, vocab=4096)
    m = qa.Model(shape, n_layers=1)
    ct = qa.QA_CACHE_F16 if cache == "f16" else qa.QA_CACHE_F32
    for cap in EDGES:
        with qa.Decoder(m, 1, cap, ct) as d:
            d.set_persistent(True)


def test_persistent_decode_streams_matches_eager(qa):
    """qa_decoder_decode_streams with one stream (the bench's decode loop) takes the persistent step too."""
    m = qa.Model(qa.QWEN3_ASR_1_7B, n_layers=2)
    x = qa.prompt_input(m, 24, 6)
    out = []
    for persistent in (False, True):
        with qa.Decoder(m, 1, 64, qa.QA_CACHE_F16) as d:
            if persistent:
                d.set_persistent(True)
            first = int(np.argmax(d.forward(x, 0)))
            ids = d.decode_streams(np.array([first], np.int32), 20)
            out.append((ids[:, 0].tolist(), d.device_lens().tolist(), d.cur_len(0)))
    assert out[1] == out[0] and out[0][1] == [50] and out[0][2] == 50


def test_persistent_step_refuses_uncovered_configs(qa):
    m = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=2)
    with qa.Decoder(m, 2, 36) as d:                  # more than one stream
        with pytest.raises(qa.QaError) as e:
            d.set_persistent(True)
        assert e.value.code == qa.QA_ERR_INVALID and "single-stream" in str(e.value)
    # a shape with no persistent kernel (intermediate 4096): refused, and the decoder stays eager and correct
    odd = qa.Model(qa.ModelSize("custom", hidden=1024, intermediate=4096, vocab=4096), n_layers=2)
    x = qa.prompt_input(odd, 24, 6)
    with qa.Decoder(odd, 1, 36) as d:
        with pytest.raises(qa.QaError) as e:
            d.set_persistent(True)
        assert e.value.code == qa.QA_ERR_INVALID and "no kernel" in str(e.value)
        ids = d.generate(x, 4)["ids"]
    with qa.Decoder(odd, 1, 36) as d:
        assert d.generate(x, 4)["ids"] == ids


def test_persistent_step_gives_up_and_recovers(qa, monkeypatch):
    """A wait bound of zero ticks (set from the host) makes the workgroups abandon the launch at a barrier:
    every kernel still ends, the call reports QA_ERR_DEVICE, and the decoder clears its barrier and merge
    state, so the next persistent generation equals the eager one."""
    m = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=2)
    x = qa.prompt_input(m, 24, 6)
    with qa.Decoder(m, 1, 36) as d:
        ref = d.generate(x, 6)["ids"]
    with qa.Decoder(m, 1, 36) as d:
        monkeypatch.setenv("QA_PERSIST_WAIT_TICKS", "0")
        d.set_persistent(True)
        with pytest.raises(qa.QaError) as e:
            d.generate(x, 6)
        assert e.value.code == qa.QA_ERR_DEVICE and "barrier" in str(e.value)
        monkeypatch.delenv("QA_PERSIST_WAIT_TICKS")
        d.set_persistent(True)
        assert d.generate(x, 6)["ids"] == ref
        d.set_persistent(False)
        assert d.generate(x, 6)["ids"] == ref
