"""CPU checks of the host-side formats around the path: the GGUF v3 writer and reader (row f3), the ASR
prompt text, the audio-token count and the WAV header (row f4, and the driver's positional WAV).

The GGUF bytes are checked by a parser written here from the GGUF specification, not by the library's
own reader, so a writer and reader that agree on a wrong layout would still fail."""
import os
import struct
import subprocess
import wave

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
WEIGHTS_TOOL = os.path.join(ROOT, "qwenasr.cpp_amd", "qwen-asr-weights")


def kv_lines(text):
    return dict(line.split("=", 1) for line in text.strip().splitlines() if "=" in line)


# ---------------------------------------------------------------------------------------------- GGUF
def parse_gguf(path):
    """GGUF v3 from the specification: header, typed key/values, tensor infos, aligned data section."""
    data = open(path, "rb").read()
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from("<" + fmt, data, pos)
        pos += struct.calcsize("<" + fmt)
        return v[0] if len(v) == 1 else v

    def string():
        nonlocal pos
        n = take("Q")
        s = data[pos:pos + n].decode()
        pos += n
        return s

    scalar = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}

    def value(t):
        if t == 8:
            return string()
        if t == 9:
            et, n = take("I"), take("Q")
            return [value(et) for _ in range(n)]
        return take(scalar[t])

    assert data[:4] == b"GGUF"
    pos = 4
    version, n_tensors, n_kv = take("I"), take("Q"), take("Q")
    kv, types = {}, {}
    for _ in range(n_kv):
        key = string()
        t = take("I")
        types[key] = t
        kv[key] = value(t)
    tensors = []
    for _ in range(n_tensors):
        name = string()
        nd = take("I")
        ne = [take("Q") for _ in range(nd)]
        tensors.append(dict(name=name, ne=ne, type=take("I"), offset=take("Q")))
    align = kv.get("general.alignment", 32)
    data_offset = (pos + align - 1) // align * align
    return dict(version=version, kv=kv, types=types, tensors=tensors, data_offset=data_offset, data=data, align=align)


def test_weights_tool_self_test():
    """The reference's fixture self-test (tools/qwen-asr-weights.cpp:58-143): write one 4-element f32
    tensor, open it back through the mapped reader, same values, shape and byte count."""
    r = subprocess.run([WEIGHTS_TOOL, "--self-test"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    kv = kv_lines(r.stdout)
    assert kv["status"] == "self-test-ok" and kv["tensors"] == "1"
    assert kv["tensor.0.name"] == "fixture.weight" and kv["tensor.0.shape"] == "[4]"
    assert kv["tensor.0.bytes"] == "16" and kv["tensor.0.offset"] == "0" and kv["tensor.0.first_f32"] == "1.25"
    assert int(kv["data_offset"]) % 32 == 0 and int(kv["file_size"]) == int(kv["data_offset"]) + 32


@pytest.fixture(scope="module")
def tiny_gguf(tmp_path_factory, qa):
    model = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=2, vocab=1000)
    path = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    model.write_gguf(path)
    return model, path


def test_gguf_writer_layout_follows_the_spec(tiny_gguf):
    model, path = tiny_gguf
    g = parse_gguf(path)
    c = model.cfg
    assert g["version"] == 3
    kv, types = g["kv"], g["types"]
    # the metadata the reference's loader requires (native-model.cpp:188-218), with their GGUF types
    assert kv["qwen3-asr.arch"] == "qwen3-asr" and types["qwen3-asr.arch"] == 8
    for key, want in (("vocab_size", c.vocab), ("hidden_size", c.hidden), ("intermediate_size", c.intermediate),
                      ("num_hidden_layers", c.n_layers), ("num_attention_heads", c.n_heads),
                      ("num_key_value_heads", c.n_kv_heads), ("head_dim", c.head_dim)):
        assert kv[f"qwen3-asr.text.{key}"] == want and types[f"qwen3-asr.text.{key}"] == 4, key
    assert kv["qwen3-asr.text.rope_theta"] == np.float32(1e6) and types["qwen3-asr.text.rope_theta"] == 6
    assert kv["qwen3-asr.text.rms_norm_eps"] == np.float32(1e-6)
    for key in ("audio.sample_rate", "audio.num_mel_bins", "audio.d_model", "audio.encoder_layers",
                "audio.encoder_attention_heads", "audio.encoder_ffn_dim", "audio.downsample_hidden_size",
                "audio.output_dim", "token.endoftext_token_id", "token.im_start_token_id", "token.im_end_token_id",
                "token.audio_token_id", "token.audio_start_token_id", "token.audio_end_token_id",
                "token.asr_text_token_id"):
        assert types[f"qwen3-asr.{key}"] == 4, key
    # a 1000-token synthetic vocabulary holds the seven special tokens at its last ids, in enum order
    specials = ["endoftext", "im_start", "im_end", "audio_start", "audio_end", "audio", "asr_text"]
    assert [kv[f"qwen3-asr.token.{n}_token_id"] for n in specials] == list(range(993, 1000))
    assert kv["tokenizer.ggml.eos_token_id"] == kv["qwen3-asr.token.im_end_token_id"] == 995
    assert kv["tokenizer.ggml.tokens"][998] == "<|audio_pad|>" and kv["tokenizer.ggml.token_type"][998] == 4
    assert kv["tokenizer.ggml.tokens"][5] == "<|unused-5|>" and kv["tokenizer.ggml.token_type"][5] == 5
    assert len(kv["tokenizer.ggml.tokens"]) == c.vocab and len(kv["tokenizer.ggml.token_type"]) == c.vocab
    assert kv["tokenizer.ggml.model"] == "gpt2" and kv["tokenizer.ggml.merges"] == ["a b"]
    # tensors: the loader's names, GGML ne order [in, out], f32, aligned increasing offsets, exact bytes
    names = {t["name"]: t for t in g["tensors"]}
    assert len(names) == 11 * c.n_layers + 3
    assert names["text.blk.1.attn_q.weight"]["ne"] == [c.hidden, 16 * 128]
    assert names["text.blk.0.attn_output.weight"]["ne"] == [16 * 128, c.hidden]
    assert names["text.blk.0.ffn_down.weight"]["ne"] == [c.intermediate, c.hidden]
    assert names["text.token_embd.weight"]["ne"] == [c.hidden, c.vocab]
    assert names["text.blk.0.attn_k_norm.weight"]["ne"] == [128]
    end = 0
    for t in g["tensors"]:
        assert t["type"] == 0 and t["offset"] % g["align"] == 0 and t["offset"] >= end, t["name"]
        n = int(np.prod(t["ne"])) * 4
        end = t["offset"] + n
        got = np.frombuffer(g["data"], np.float32, n // 4, g["data_offset"] + t["offset"])
        np.testing.assert_array_equal(got, model.tensor(t["name"]), err_msg=t["name"])
    assert len(g["data"]) >= g["data_offset"] + end


def test_gguf_reader_opens_writer_output(tiny_gguf):
    model, path = tiny_gguf
    r = subprocess.run([WEIGHTS_TOOL, path, "--tensor", "text.blk.1.ffn_gate.weight"], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    kv = kv_lines(r.stdout)
    g = parse_gguf(path)
    assert int(kv["tensors"]) == len(g["tensors"]) and int(kv["data_offset"]) == g["data_offset"]
    assert kv["tensor.shape"] == f"[{model.cfg.hidden},{model.cfg.intermediate}]"
    assert np.float32(kv["tensor.first_f32"]) == pytest.approx(model.tensor("text.blk.1.ffn_gate.weight")[0], rel=1e-5)
    r = subprocess.run([WEIGHTS_TOOL, path, "--tensor", "text.blk.9.attn_q.weight"], capture_output=True, text=True)
    assert r.returncode == 1 and "missing GGUF tensor: text.blk.9.attn_q.weight" in r.stderr


def test_gguf_reader_rejects_damaged_files(tiny_gguf, tmp_path):
    _, path = tiny_gguf
    data = open(path, "rb").read()
    cut = tmp_path / "cut.gguf"
    cut.write_bytes(data[: len(data) - 4096])
    r = subprocess.run([WEIGHTS_TOOL, str(cut)], capture_output=True, text=True)
    assert r.returncode == 1 and "tensor data extends beyond GGUF file" in r.stderr
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + data[4:4096])
    r = subprocess.run([WEIGHTS_TOOL, str(bad)], capture_output=True, text=True)
    assert r.returncode == 1 and "bad magic" in r.stderr


# ---------------------------------------------------------------------------------------------- prompt
def test_asr_prompt_layout(qa):
    """qwenasr_build_asr_prompt (tokenizer.cpp:529-549): the chat turns of the Qwen3-ASR template with
    one <|audio_pad|> per audio-encoder row between <|audio_start|> and <|audio_end|>, and the forced
    language suffix only when a language is given."""
    p = qa.build_asr_prompt(3, "Be brief.", "English")
    head, rest = p.split("<|audio_start|>")
    assert head == "<|im_start|>system\nBe brief.<|im_end|>\n<|im_start|>user\n"
    pads, tail = rest.split("<|audio_end|>")
    assert pads == "<|audio_pad|>" * 3
    assert tail == "<|im_end|>\n<|im_start|>assistant\nlanguage English<asr_text>"
    plain = qa.build_asr_prompt(143)
    assert plain.count("<|audio_pad|>") == 143 and plain.endswith("<|im_start|>assistant\n")
    assert "language" not in plain and "<asr_text>" not in plain
    assert plain.startswith("<|im_start|>system\n<|im_end|>\n")
    assert qa.build_asr_prompt(-5) == qa.build_asr_prompt(0) and "<|audio_pad|>" not in qa.build_asr_prompt(0)
    # the length grows by exactly one placeholder per audio row
    assert len(qa.build_asr_prompt(10)) - len(qa.build_asr_prompt(9)) == len("<|audio_pad|>")


def test_audio_output_length_matches_hf_processor(qa):
    """The audio-encoder output length (audio-features.cpp:14-19) against transformers' Qwen3-ASR
    processor formula (_get_audio_token_length, n_window 50), a library routine, for 0..5000 frames."""
    torch = pytest.importorskip("torch")
    proc = pytest.importorskip("transformers.models.qwen3_asr.processing_qwen3_asr")
    frames = np.arange(1, 5001)
    ref = proc.Qwen3ASRProcessor._get_audio_token_length(None, torch.from_numpy(frames))
    got = np.array([qa.lib.qa_audio_output_length(int(f)) for f in frames])
    np.testing.assert_array_equal(got, ref)
    assert qa.lib.qa_audio_output_length(1100) == 143        # the 11 s clip of the reference's README: 143 rows
    assert qa.lib.qa_audio_output_length(0) == 0


def _write_wav(path, n, rate=16000, width=2, channels=1):
    with wave.open(str(path), "wb") as w:
        w.setnchannels(channels)
        w.setsampwidth(width)
        w.setframerate(rate)
        w.writeframes(bytes(width * n * channels))


def test_wav_info_counts_sample_frames(qa, tmp_path):
    p = tmp_path / "a.wav"
    _write_wav(p, 176000)
    assert qa.wav_info(str(p)) == (176000, 16000)
    _write_wav(p, 1000, channels=2)                           # frames, not samples, of a stereo file
    assert qa.wav_info(str(p)) == (1000, 16000)
    _write_wav(p, 4800, width=3)
    assert qa.wav_info(str(p)) == (4800, 16000)
    _write_wav(p, 100, rate=44100)
    with pytest.raises(qa.QaError, match="16 kHz"):
        qa.wav_info(str(p))
    with pytest.raises(qa.QaError, match="failed to open WAV"):
        qa.wav_info(str(tmp_path / "missing.wav"))
