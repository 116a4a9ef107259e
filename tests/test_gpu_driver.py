"""The text-layer driver run with the reference harness's command lines on the GPU, and the non-cached
entry points (qwenasr_text_layer_backend_forward / qwenasr_text_prefill_backend_forward,
text-decoder.cpp:1305-1390 and 1757-1854) against the oracle.

The harness parses stdout with _parse_kv and indexes generate_ms, prefill_ms, text_layer_ms,
decoder_input_ms, text_init_ms, backend, audio_backend, decode_backend, stopped, generated_ids,
text_json, tokens, hidden and vocab (benchmarks/bench_text_*.py, check_text_*.py); every one of them is
read here the way the harness reads it."""
import json
import os
import subprocess
import wave

import numpy as np
import pytest
from test_driver import TOOL, harness_generate_argv, parse_kv

pytestmark = pytest.mark.gpu


def close(got, ref, atol, rtol_l2):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    err = float(np.abs(got - ref).max())
    rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    assert err <= atol and rel <= rtol_l2, (err, rel)


@pytest.fixture(scope="module", autouse=True)
def _gpu(qa):
    assert qa.device_count() > 0, "no HIP device: GPU tests need the MI355X"


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory, qa, orc):
    d = tmp_path_factory.mktemp("gpu_driver")
    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=2, vocab=2048)
    gguf = d / "model.gguf"
    model.write_gguf(str(gguf))
    wav = d / "clip.wav"
    with wave.open(str(wav), "wb") as w:
        w.setnchannels(1)
        w.setsampwidth(2)
        w.setframerate(16000)
        w.writeframes(bytes(2 * 176000))          # 11 s -> 143 audio rows, plus 13 prompt ids
    om = orc.OracleModel.from_product_model(model)
    x = qa.prompt_input(model, 143, 13)           # the driver's decoder input for this clip and seed
    return model, om, x, gguf, wav, d


def run(cmd):
    print("run:", " ".join(map(str, cmd[1:])), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    return parse_kv(r.stdout)


def test_harness_generate_command(checkpoint):
    model, om, x, gguf, wav, _ = checkpoint
    n = 8
    meta = run(harness_generate_argv(gguf, wav, n, system="Transcribe.", language="English"))
    for key in ("generate_ms", "decoder_input_ms", "text_init_ms"):
        assert float(meta[key]) >= 0.0, key
    assert meta["backend"] == "sched" and meta["audio_backend"] == "sched" and meta["decode_backend"] == "kv-cache"
    ids = [int(v) for v in meta["generated_ids"].split(",") if v]
    assert json.loads(meta["text_json"]) == meta["generated_ids"]
    assert int(meta["prompt_tokens"]) == 156 and int(meta["feature_frames"]) == 1100
    # stop ids of this checkpoint: im_end, endoftext, eos (tools/qwen-asr-text-layer.cpp:395-399)
    stops = [model.cfg.vocab - 5, model.cfg.vocab - 7, model.cfg.vocab - 5]
    ref = om.generate(x, n, stops, om.cache(156 + n, f16=False))      # the reference's f32 cache
    assert ids == ref["ids"], (ids, ref["ids"], ref["margins"])
    assert meta["stopped"] == ("true" if ref["stopped"] else "false")
    assert int(meta["total_tokens"]) == ref["total_tokens"] and int(meta["generated_tokens"]) == len(ids)


def test_harness_generate_command_persistent(checkpoint):
    """The same harness command with QA_DECODE_PERSISTENT=1 in the environment: the drop-in's decoder runs each
    decode step as one persistent launch, and the generated ids are the oracle's (and the eager run's)."""
    model, om, x, gguf, wav, _ = checkpoint
    n = 8
    env = dict(os.environ, QA_DECODE_PERSISTENT="1")
    cmd = harness_generate_argv(gguf, wav, n, system="Transcribe.", language="English")
    print("run:", " ".join(map(str, cmd[1:])), "(QA_DECODE_PERSISTENT=1)", flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stderr
    meta = parse_kv(r.stdout)
    ids = [int(v) for v in meta["generated_ids"].split(",") if v]
    stops = [model.cfg.vocab - 5, model.cfg.vocab - 7, model.cfg.vocab - 5]
    ref = om.generate(x, n, stops, om.cache(156 + n, f16=False))
    assert ids == ref["ids"], (ids, ref["ids"], ref["margins"])


def test_harness_generate_command_bf16_checkpoint(tmp_path, qa, orc, greedy):
    """A GGUF holding bf16-exact weights (what the reference's converter writes from the released bf16
    checkpoint, convert.py:386-387) through the drop-in: the decoder keeps bf16 weight copies and the
    generated ids still match the oracle's on the same f32 values."""
    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=2, vocab=2048, bf16=True)
    gguf = tmp_path / "model_bf16.gguf"
    model.write_gguf(str(gguf))
    wav = tmp_path / "clip.wav"
    with wave.open(str(wav), "wb") as w:
        w.setnchannels(1)
        w.setsampwidth(2)
        w.setframerate(16000)
        w.writeframes(bytes(2 * 176000))
    n = 8
    meta = run(harness_generate_argv(gguf, wav, n))
    ids = [int(v) for v in meta["generated_ids"].split(",") if v]
    om = orc.OracleModel.from_product_model(model)
    x = qa.prompt_input(model, 143, 13)
    stops = [model.cfg.vocab - 5, model.cfg.vocab - 7, model.cfg.vocab - 5]
    ref = om.generate(x, n, stops, om.cache(156 + n, f16=False))
    assert greedy.match(ids, ref["ids"], ref["margins"], ref["runner_up"],
                        "driver generate, bf16-exact GGUF (f32 cache)") is None


def test_harness_prefill_command(checkpoint):
    """check_text_prefill.py:37-60: --prefill --out logits.f32, file shape (vocab,) against the oracle's
    non-cached prefill."""
    model, om, x, gguf, wav, d = checkpoint
    out = d / "logits.f32"
    meta = run([TOOL, str(gguf), str(wav), "--threads", "8", "--backend", "sched", "--audio-backend", "sched",
                "--device", "auto", "--prefill", "--out", str(out)])
    values = np.fromfile(out, dtype=np.float32)
    assert values.shape == (int(meta["vocab"]),) and float(meta["prefill_ms"]) > 0 and float(meta["decoder_input_ms"]) >= 0
    assert int(meta["tokens"]) == 156 and int(meta["hidden"]) == model.cfg.hidden
    close(values, om.prefill_nocache(x), atol=2e-3, rtol_l2=1e-3)
    assert int(meta["top_id"]) == int(np.argmax(values))


def test_harness_layer_command(checkpoint):
    """check_text_layer0.py:33-57: --layer N --out values.f32, reshaped [tokens][hidden], against the
    oracle's non-cached layer."""
    model, om, x, gguf, wav, d = checkpoint
    out = d / "layer.f32"
    meta = run([TOOL, str(gguf), str(wav), "--threads", "8", "--backend", "sched", "--audio-backend", "ggml",
                "--device", "auto", "--layer", "1", "--out", str(out)])
    values = np.fromfile(out, dtype=np.float32).reshape(int(meta["tokens"]), int(meta["hidden"]))
    assert float(meta["text_layer_ms"]) > 0 and meta["audio_backend"] == "ggml" and meta["backend"] == "sched"
    close(values, om.layer_forward_nocache(1, x), atol=1e-4, rtol_l2=1e-5)


@pytest.fixture(scope="module")
def small(qa, orc):
    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=2)
    return model, orc.OracleModel.from_product_model(model)


@pytest.mark.parametrize("T", [5, 156, 1024])
def test_nocache_entry_points_match_oracle(qa, small, T):
    """qa_decoder_layer_forward_nocache and qa_decoder_prefill_nocache (positions 0..T-1, f32 K/V never
    stored) at T = 5 (skinny MFMA projections), 156 and 1024 (rocBLAS projections), against
    orc_layer_forward_nocache / the oracle's non-cached prefill; the cache is left untouched."""
    model, om = small
    x = qa.prompt_input(model, T - 3, 3)
    with qa.Decoder(model, 1, 8, qa.QA_CACHE_F32) as dec:
        for layer in (0, 1):
            close(dec.layer_forward_nocache(layer, x), om.layer_forward_nocache(layer, x), atol=1e-4, rtol_l2=1e-5)
        close(dec.prefill_nocache(x), om.prefill_nocache(x), atol=2e-3, rtol_l2=1e-3)
        ptr, lay = dec.cache()
        n = lay.n_layers * 2 * lay.n_streams * lay.n_kv_heads * lay.max_seq * lay.head_dim
        cache = np.empty(n, np.float32)
        qa.check(qa.lib.qa_copy_to_host(cache.ctypes.data, ptr, n * 4))
        assert not cache.any() and dec.cur_len(0) == 0
