"""The text-layer driver against the reference harness's command lines, on the CPU.

benchmarks/bench_text_generate.py:44-65 (and bench_text_prefill.py, bench_text_layer0.py,
check_text_*.py) run the tool as `tool model.gguf audio.wav --threads N --backend B --audio-backend A
--device D ...` and parse its stdout with _parse_kv (check_audio_conv0.py:20-26).  Without a GPU the
driver must get through argument parsing, the GGUF checkpoint, the WAV and the decoder input, and stop
at the device: exit 1, not the argument error (exit 2).  The GPU run of the same command lines is in
test_gpu_driver.py."""
import os
import subprocess
import wave

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOOL = os.path.join(ROOT, "qwenasr.cpp_amd", "qwen-asr-text-layer")


def parse_kv(text):
    """The harness's parser (benchmarks/check_audio_conv0.py:20-26): key=value lines, stripped."""
    out = {}
    for line in text.splitlines():
        if "=" in line:
            k, v = line.split("=", 1)
            out[k.strip()] = v.strip()
    return out


def harness_generate_argv(gguf, wav, n, system="", language="", device="auto"):
    """bench_text_generate.py:44-63 with text backend sched, audio backend sched, decode backend kv-cache."""
    cmd = [TOOL, str(gguf), str(wav), "--threads", "8", "--backend", "sched", "--audio-backend", "sched",
           "--device", device, "--generate", str(n), "--kv-cache"]
    if system:
        cmd += ["--system", system]
    if language:
        cmd += ["--language", language]
    return cmd


@pytest.fixture(scope="module")
def inputs(tmp_path_factory, qa):
    d = tmp_path_factory.mktemp("driver")
    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=2, vocab=2048)
    gguf = d / "model.gguf"
    model.write_gguf(str(gguf))
    wav = d / "clip.wav"
    with wave.open(str(wav), "wb") as w:
        w.setnchannels(1)
        w.setsampwidth(2)
        w.setframerate(16000)
        w.writeframes(bytes(2 * 176000))         # 11 s: 1100 mel frames -> 143 audio rows
    return model, gguf, wav


def run(cmd, **kw):
    return subprocess.run(cmd, capture_output=True, text=True, timeout=300, **kw)


@pytest.mark.skipif(os.environ.get("HIP_VISIBLE_DEVICES") is None and os.path.exists("/dev/kfd"),
                    reason="a GPU is visible: the full run is test_gpu_driver.py")
def test_harness_argv_reaches_the_device_step(inputs):
    _, gguf, wav = inputs
    for cmd in (harness_generate_argv(gguf, wav, 4),
                harness_generate_argv(gguf, wav, 4, system="Transcribe.", language="English"),
                [TOOL, str(gguf), str(wav), "--threads", "8", "--backend", "sched", "--audio-backend", "sched",
                 "--device", "auto", "--prefill", "--out", os.devnull],
                [TOOL, str(gguf), str(wav), "--threads", "8", "--backend", "sched", "--audio-backend", "ggml",
                 "--device", "auto", "--layer", "1", "--out", os.devnull]):
        r = run(cmd)
        assert r.returncode == 1, (cmd, r.returncode, r.stderr)
        assert "HIP" in r.stderr or "device" in r.stderr, r.stderr


def test_reference_argument_errors(inputs):
    """Exit 2 with the reference tool's messages (tools/qwen-asr-text-layer.cpp:95-272)."""
    _, gguf, wav = inputs
    cases = [
        ([str(gguf)], "model GGUF and audio WAV are required"),
        ([str(gguf), str(wav), "--prefill", "--generate", "2"], "--prefill and --generate are mutually exclusive"),
        ([str(gguf), str(wav), "--backend", "scalar", "--kv-cache"], "--kv-cache requires --generate"),
        ([str(gguf), str(wav), "--backend", "ggml", "--generate", "2"], "--backend ggml currently supports layer mode only"),
        ([str(gguf), str(wav), "--backend", "ggml", "--prefill"], "--backend ggml currently supports layer mode only"),
        ([str(gguf), str(wav), "extra"], "too many positional arguments"),
        ([str(gguf), str(wav), "--backend", "fast"], "--backend requires scalar, ggml, or sched"),
        ([str(gguf), str(wav), "--audio-backend", "x"], "--audio-backend requires ggml or sched"),
        ([str(gguf), str(wav), "--generate", "2000"], "--generate requires a non-negative integer up to 1024"),
        ([str(gguf), str(wav), "--threads", "0"], "--threads requires a positive integer"),
        ([str(gguf), str(wav), "--layer", "-1"], "--layer requires a non-negative integer"),
        ([str(gguf), str(wav), "--device", "tpu"], "device"),
        ([str(gguf), str(wav), "--layer", "2"], "--layer is out of range for model"),
    ]
    for args, msg in cases:
        r = run([TOOL] + args)
        assert r.returncode == 2 and msg in r.stderr, (args, r.returncode, r.stderr)


def test_cpu_backends_and_inputs_fail_cleanly(inputs, tmp_path):
    """The reference's scalar/ggml CPU paths are not shipped: exit 1 with an error, never a silent CPU
    run.  Missing and malformed inputs give the reference's errors (exit 1)."""
    _, gguf, wav = inputs
    r = run([TOOL, str(gguf), str(wav), "--backend", "scalar", "--generate", "2"])
    assert r.returncode == 1 and "not part of the MI355X build" in r.stderr, r.stderr
    r = run([TOOL, str(gguf), str(wav), "--backend", "ggml", "--layer", "0"])
    assert r.returncode == 1 and "not part of the MI355X build" in r.stderr, r.stderr
    r = run([TOOL, str(tmp_path / "missing.gguf"), str(wav), "--generate", "2"])
    assert r.returncode == 1 and "failed to open GGUF file" in r.stderr
    r = run([TOOL, str(gguf), str(tmp_path / "missing.wav"), "--generate", "2"])
    assert r.returncode == 1 and "failed to open WAV" in r.stderr
    slow = tmp_path / "44k.wav"
    with wave.open(str(slow), "wb") as w:
        w.setnchannels(1)
        w.setsampwidth(2)
        w.setframerate(44100)
        w.writeframes(bytes(2000))
    r = run([TOOL, str(gguf), str(slow), "--generate", "2"])
    assert r.returncode == 1 and "requires 16 kHz WAV input" in r.stderr
