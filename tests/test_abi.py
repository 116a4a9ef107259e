"""CPU checks of the C-ABI library and the C++ drop-in: symbols, generator, layout, host errors."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "qwenasr.cpp_amd", "libqwenasr_amd.so")
TOOL = os.path.join(ROOT, "qwenasr.cpp_amd", "qwen-asr-text-layer")


def header_functions(name):
    text = open(os.path.join(ROOT, "include", name)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b((?:qa|qwenasr)_[a-z0-9_]+)\s*\(", text)))


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", LIB], capture_output=True, text=True, check=True).stdout
    return out


def test_c_abi_exports_every_declared_symbol(qa):
    names = header_functions("qwenasr_amd.h")
    assert len(names) > 50
    syms = exported()
    for n in names:
        assert re.search(rf" T {n}$", syms, re.M), n
        assert hasattr(qa.lib, n)
    assert set(names) == set(qa.SIGNATURES), set(names) ^ set(qa.SIGNATURES)


@pytest.mark.parametrize("header", ["text-decoder.h", "ggml-backends.h", "gguf-model.h", "decoder-input.h",
                                    "tokenizer.h"])
def test_cpp_drop_in_exports(header):
    syms = exported()
    names = header_functions(header)
    assert names
    for n in names:
        assert re.search(rf" T {n}\(", syms), n
    if header == "text-decoder.h":   # the reference's 13 functions (src/text-decoder.h:35-179) plus 2 additions
        assert len([n for n in names if n.startswith("qwenasr_text_")]) == 15


def test_generator_kat_and_properties(qa):
    # splitmix64 seeded with 1234567: the published first outputs
    assert [qa.lib.qa_synth_word(1234567, i) for i in range(3)] == [6457827717110365317, 3203168211198807973,
                                                                     9817491932198370423]
    a = qa.synth_normal(1 << 20, 7, "w", 0.02)
    b = qa.synth_normal(1 << 20, 7, "w", 0.02)
    np.testing.assert_array_equal(a, b)
    assert abs(a.mean()) < 1e-4 and abs(a.std() - 0.02) < 1e-4
    head = qa.synth_normal(1000, 7, "w", 0.02)
    np.testing.assert_array_equal(head, a[:1000])          # element j depends only on (seed, name, j)
    assert not np.array_equal(qa.synth_normal(1000, 7, "v", 0.02), head)
    ids = qa.synth_ids(100000, 9, "ids", 156, 3913)
    assert ids.min() >= 156 and ids.max() <= 3913 and len(np.unique(ids)) > 3000


def test_layout_bookkeeping(qa):
    lay = qa.KvLayout(28, 1, 8, 128, 4169, qa.QA_CACHE_F16)
    assert qa.lib.qa_kv_cache_bytes(C.byref(lay)) == 28 * 2 * 8 * 4169 * 128 * 2
    assert qa.lib.qa_kv_cache_bytes(C.byref(lay)) // 4169 == 114688            # 114 KB per position
    assert qa.lib.qa_kv_slot_index(C.byref(lay), 27, 1, 0, 7, 4168, 127) == 28 * 2 * 8 * 4169 * 128 - 1
    assert qa.lib.qa_kv_slot_index(C.byref(lay), 0, 0, 0, 0, 4169, 0) == -1
    lay4 = qa.KvLayout(28, 32, 8, 128, 3977, qa.QA_CACHE_F16)
    idx = qa.lib.qa_kv_slot_index(C.byref(lay4), 3, 1, 17, 5, 100, 9)
    assert idx == ((((3 * 2 + 1) * 32 + 17) * 8 + 5) * 3977 + 100) * 128 + 9
    bad = qa.KvLayout(0, 1, 8, 128, 10, 0)
    assert qa.lib.qa_kv_layout_check(C.byref(bad)) == qa.QA_ERR_INVALID
    assert "KV-cache" in qa.lib.qa_last_error().decode()


def test_no_device_errors_are_loud(qa):
    if qa.device_count() > 0:
        pytest.skip("a GPU is visible")
    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=1, vocab=64)
    with pytest.raises(qa.QaError) as e:
        qa.Decoder(model, 1, 16)
    assert e.value.code == qa.QA_ERR_NO_DEVICE
    r = subprocess.run([TOOL, "--size", "0.6b", "--layers", "1", "--generate", "2"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 1 and "no HIP device" in r.stderr


def test_tool_argument_errors():
    r = subprocess.run([TOOL, "--size", "0.6b", "--prefill", "--generate", "2"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 2 and "mutually exclusive" in r.stderr
    r = subprocess.run([TOOL, "--generate", "2000"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "up to 1024" in r.stderr
    r = subprocess.run([TOOL, "--device", "tpu"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "auto, cpu, gpu, or cuda" in r.stderr


def test_decoder_input_assembly(qa):
    """qwenasr_decoder_input_from_audio after tokenization (decoder-input.cpp:26-101): embedding rows of
    the prompt ids, the i-th audio placeholder replaced by audio row i; errors before any write."""
    vocab, hidden, pad = 50, 16, 7
    rng = np.random.default_rng(3)
    embd = rng.standard_normal((vocab, hidden)).astype(np.float32)
    audio = rng.standard_normal((4, hidden)).astype(np.float32)
    ids = np.array([1, 2, 3, pad, pad, pad, pad, 4, 5, 49, 0], np.int32)
    out = np.zeros((len(ids), hidden), np.float32)

    def run(ids, audio, out, audio_token_id=pad, vocab=vocab):
        return qa.lib.qa_decoder_input_assemble(embd.ctypes.data, vocab, hidden, ids.ctypes.data, len(ids),
                                                audio_token_id, audio.ctypes.data, len(audio), out.ctypes.data)

    assert run(ids, audio, out) == qa.QA_OK
    expect = embd[ids].copy()
    expect[3:7] = audio
    np.testing.assert_array_equal(out.view(np.uint32), expect.view(np.uint32))
    cases = [
        (np.array([1, pad, pad, 2], np.int32), audio, "audio placeholder count does not match"),
        (np.array([pad] * 5, np.int32), audio, "more audio placeholders than audio encoder outputs"),
        (np.array([1, pad, pad, pad, pad, vocab], np.int32), audio, "out of embedding range"),
        (np.array([-1, pad, pad, pad, pad], np.int32), audio, "out of embedding range"),
    ]
    for bad_ids, a, msg in cases:
        sentinel = np.full((len(bad_ids), hidden), 7.5, np.float32)
        assert run(bad_ids, a, sentinel) == qa.QA_ERR_INVALID
        assert msg in qa.lib.qa_last_error().decode(), msg
        assert (sentinel == 7.5).all()                     # nothing written on error
    assert run(ids, audio, out, audio_token_id=-1) == qa.QA_ERR_INVALID
    assert "invalid decoder input configuration" in qa.lib.qa_last_error().decode()
    empty = np.zeros((0,), np.int32)
    assert qa.lib.qa_decoder_input_assemble(embd.ctypes.data, vocab, hidden, empty.ctypes.data, 0, pad,
                                            audio.ctypes.data, len(audio), out.ctypes.data) == qa.QA_ERR_INVALID
    assert "no tokens" in qa.lib.qa_last_error().decode()
