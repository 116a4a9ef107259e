"""Host-side Python binding of the MI355X Qwen3-ASR text-decoder KV-cache path.

Everything here goes through the C ABI of ``include/qwenasr_amd.h`` (``libqwenasr_amd.so``, built by
``make`` in ``qwenasr.cpp_amd/``).  The binding mirrors the reference's text-decoder.h contract
(src/text-decoder.h:10-179 of andimarafioti/qwenasr.cpp): a decoder backend owns the weights and the
KV cache, ``forward`` is one cached call (text_decoder_backend_cached_logits, text-decoder.cpp:1641-1755)
and ``generate`` is qwenasr_text_generate_cached_backend (text-decoder.cpp:2209-2311).

Importing this module never falls back to anything: if the shared library is missing the import
fails with the command that builds it.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "libqwenasr_amd.so")

QA_OK, QA_ERR_INVALID, QA_ERR_CAPACITY, QA_ERR_DEVICE, QA_ERR_NO_DEVICE, QA_ERR_ALLOC, QA_ERR_RANGE = range(7)
QA_CACHE_F32, QA_CACHE_F16 = 0, 1
QA_NOALLOC_SCRATCH_BYTES = 48 << 20   # include/qwenasr_amd.h


class QaError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is not built; run `make -C {_PKG_DIR}` (or __graft_entry__.build())"
    )
lib = C.CDLL(LIB_PATH)

i32, i64, u64, f32, sz = C.c_int32, C.c_int64, C.c_uint64, C.c_float, C.c_size_t
vp, fp, ip = C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_int32)


class TextConfig(C.Structure):
    _fields_ = [("n_layers", i32), ("hidden", i32), ("n_heads", i32), ("n_kv_heads", i32), ("head_dim", i32),
                ("intermediate", i32), ("vocab", i32), ("rope_theta", f32), ("rms_norm_eps", f32)]


class KvLayout(C.Structure):
    _fields_ = [("n_layers", i32), ("n_streams", i32), ("n_kv_heads", i32), ("head_dim", i32), ("max_seq", i32),
                ("cache_type", i32)]


class LayerWeights(C.Structure):
    _fields_ = [(n, fp) for n in ("attn_norm", "ffn_norm", "q", "k", "v", "o", "q_norm", "k_norm", "gate", "up",
                                  "down")]


class ModelWeights(C.Structure):
    _fields_ = [("layers", C.POINTER(LayerWeights)), ("token_embd", fp), ("output_norm", fp), ("output", fp)]


def _sig(name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)
    return f


# every symbol declared in include/qwenasr_amd.h, with its C signature
SIGNATURES = {
    "qa_last_error": (C.c_char_p,),
    "qa_device_count": (C.c_int,),
    "qa_device_arch": (C.c_int, C.c_char_p, sz),
    "qa_copy_to_host": (C.c_int, vp, vp, sz),
    "qa_device_synchronize": (C.c_int,),
    "qa_device_malloc": (C.c_int, C.POINTER(vp), sz),
    "qa_device_free": (C.c_int, vp),
    "qa_copy_to_device": (C.c_int, vp, vp, sz),
    "qa_copy_device": (C.c_int, vp, vp, sz, vp),
    "qa_memset_device": (C.c_int, vp, C.c_int, sz),
    "qa_event_create": (C.c_int, C.POINTER(vp)),
    "qa_event_destroy": (C.c_int, vp),
    "qa_event_record": (C.c_int, vp, vp),
    "qa_event_elapsed_ms": (C.c_int, vp, vp, C.POINTER(C.c_float)),
    "qa_stream_synchronize": (C.c_int, vp),
    "qa_kv_layout_check": (C.c_int, C.POINTER(KvLayout)),
    "qa_kv_elem_bytes": (sz, i32),
    "qa_kv_cache_bytes": (sz, C.POINTER(KvLayout)),
    "qa_kv_slot_index": (i64, C.POINTER(KvLayout), i32, i32, i32, i32, i32, i32),
    "qa_kv_cache_alloc": (C.c_int, C.POINTER(KvLayout), C.POINTER(vp)),
    "qa_kv_cache_free": (C.c_int, vp),
    "qa_positions": (C.c_int, i32, i32, ip),
    "qa_causal_mask": (C.c_int, i32, i32, fp),
    "qa_kv_append": (C.c_int, vp, vp, vp, vp, vp, C.POINTER(KvLayout), i32, vp, i32, i32, i32, f32, f32, vp),
    "qa_decode_attn_workspace_bytes": (sz, i32, i32, i32),
    "qa_workspace_clear": (C.c_int, vp, sz, vp),
    "qa_decode_attn": (C.c_int, vp, vp, C.POINTER(KvLayout), i32, vp, i32, i32, i32, f32, vp, vp, sz, vp),
    "qa_decode_step_attn": (C.c_int, vp, vp, vp, vp, C.POINTER(KvLayout), i32, vp, i32, i32, i32, f32, f32, f32, vp,
                            vp, sz, vp),
    "qa_decode_step_attn_noalloc": (C.c_int, vp, vp, vp, vp, C.POINTER(KvLayout), i32, vp, i32, i32, i32, f32, f32,
                                    f32, vp, vp),
    "qa_decode_noalloc_prepare": (C.c_int,),
    "qa_prefill_attn_workspace_bytes": (sz, i32, i32),
    "qa_prefill_attn": (C.c_int, vp, vp, C.POINTER(KvLayout), i32, i32, i32, i32, i32, f32, vp, vp, sz, vp),
    "qa_causal_attn_f32": (C.c_int, vp, vp, vp, i32, i32, i32, f32, vp, vp),
    "qa_qk_prep": (C.c_int, vp, i32, i32, i32, vp, vp, i32, f32, f32, vp),
    "qa_gemv": (C.c_int, vp, i32, i32, vp, i32, vp, i32, vp),
    "qa_gemv_fused": (C.c_int, vp, vp, i32, i32, vp, vp, i32, vp, f32, vp),
    "qa_pack_bf16": (C.c_int, vp, i64, vp, vp, vp),
    "qa_rmsnorm_rows": (C.c_int, vp, vp, i32, i32, f32, vp, vp),
    "qa_swiglu_rows": (C.c_int, vp, i32, i32, vp, vp),
    "qa_add_inplace": (C.c_int, vp, vp, sz, vp),
    "qa_argmax_workspace_bytes": (sz, i32),
    "qa_argmax_rows": (C.c_int, vp, i32, i32, vp, vp, sz, vp),
    "qa_embed_rows": (C.c_int, vp, i32, i32, vp, i32, vp, vp),
    "qa_advance_lens": (C.c_int, vp, i32, i32, vp),
    "qa_synth_key": (u64, u64, C.c_char_p),
    "qa_synth_word": (u64, u64, u64),
    "qa_synth_fill_normal": (None, fp, sz, u64, C.c_char_p, C.c_double),
    "qa_synth_fill_const": (None, fp, sz, f32),
    "qa_synth_fill_ids": (None, ip, sz, u64, C.c_char_p, i32, i32),
    "qa_model_synthetic": (C.c_int, C.POINTER(TextConfig), u64, C.POINTER(vp)),
    "qa_model_round_bf16": (C.c_int, vp),
    "qa_decoder_weights_bf16": (C.c_int, vp),
    "qa_model_free": (None, vp),
    "qa_model_tensor": (fp, vp, C.c_char_p, C.POINTER(i64)),
    "qa_model_config": (C.c_int, vp, C.POINTER(TextConfig)),
    "qa_decoder_input_assemble": (C.c_int, vp, i32, i32, vp, i32, i32, vp, i32, vp),
    "qa_gguf_write_model": (C.c_int, vp, C.c_char_p),
    "qa_build_asr_prompt": (C.c_int, i32, C.c_char_p, C.c_char_p, C.c_char_p, sz, C.POINTER(sz)),
    "qa_audio_output_length": (i32, i32),
    "qa_wav_info": (C.c_int, C.c_char_p, C.POINTER(i64), C.POINTER(i32)),
    "qa_gemm_rows_workspace_bytes": (sz, i32, i32, i32),
    "qa_gemm_rows": (C.c_int, vp, i32, i32, vp, i32, vp, i32, vp, sz, vp),
    "qa_gemm_rows_fused": (C.c_int, vp, i32, i32, vp, i32, vp, i32, vp, vp, i32, f32, vp, i32, vp, sz, vp),
    "qa_gemm_rows_fused_bf16": (C.c_int, vp, i32, i32, vp, i32, vp, i32, vp, vp, i32, f32, vp, i32, vp, sz, vp),
    "qa_gemm_split3_bf16": (C.c_int, vp, i32, i32, vp, i32, vp, i32, vp, vp),
    "qa_model_weights_view": (C.c_int, vp, C.POINTER(LayerWeights), i32, C.POINTER(ModelWeights)),
    "qa_decoder_create": (C.c_int, C.POINTER(TextConfig), C.POINTER(ModelWeights), i32, i32, i32, C.POINTER(vp)),
    "qa_decoder_destroy": (None, vp),
    "qa_decoder_cur_len": (C.c_int, vp, i32, ip),
    "qa_decoder_device_lens": (C.c_int, vp, ip),
    "qa_decoder_set_cur_len": (C.c_int, vp, i32, i32),
    "qa_decoder_cache": (vp, vp, C.POINTER(KvLayout)),
    "qa_decoder_stream": (vp, vp),
    "qa_decoder_forward": (C.c_int, vp, fp, i32, i32, fp),
    "qa_decoder_generate": (C.c_int, vp, fp, i32, i32, ip, i32, ip, ip, ip, ip, fp),
    "qa_decoder_decode_streams": (C.c_int, vp, ip, i32, ip),
    "qa_decoder_set_persistent": (C.c_int, vp, i32),
    "qa_decoder_fill_cache": (C.c_int, vp, i32, fp, fp, i32),
    "qa_decoder_layer_forward": (C.c_int, vp, i32, fp, i32, i32, fp),
    "qa_decoder_layer_forward_nocache": (C.c_int, vp, i32, fp, i32, fp),
    "qa_decoder_prefill_nocache": (C.c_int, vp, fp, i32, fp),
    "qa_decoder_profile_enable": (C.c_int, vp, i32),
    "qa_decoder_profile_read": (C.c_int, vp, C.c_char_p, C.POINTER(C.c_double), C.POINTER(i64)),
    "qa_decoder_profile_reset": (C.c_int, vp),
}
for _name, (_res, *_args) in SIGNATURES.items():
    _sig(_name, _res, *_args)


def check(rc: int) -> None:
    if rc != QA_OK:
        raise QaError(rc, lib.qa_last_error().decode())


def fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(fp)


def iptr(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(ip)


def device_count() -> int:
    return lib.qa_device_count()


class DeviceArray:
    """A device buffer of device 0 owned through the C ABI (qa_device_malloc), with numpy transfers."""

    def __init__(self, shape, dtype=np.float32, zero: bool = True):
        self.shape = tuple(int(v) for v in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        h = vp()
        check(lib.qa_device_malloc(C.byref(h), self.nbytes))
        self.handle = h
        if zero:
            check(lib.qa_memset_device(self.handle, 0, self.nbytes))

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype, zero=False)
        d.upload(a)
        return d

    @property
    def ptr(self):
        return self.handle

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.shape, self.shape)
        check(lib.qa_copy_to_device(self.handle, a.ctypes.data, self.nbytes))

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        check(lib.qa_copy_to_host(out.ctypes.data, self.handle, self.nbytes))
        return out

    def free(self):
        if getattr(self, "handle", None):
            lib.qa_device_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize():
    check(lib.qa_device_synchronize())


# ----------------------------------------------------------------------------------------- model sizes
@dataclass(frozen=True)
class ModelSize:
    name: str
    hidden: int
    intermediate: int
    n_layers: int = 28
    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 151936
    rope_theta: float = 1.0e6
    rms_norm_eps: float = 1.0e-6

    def config(self, n_layers: int | None = None, vocab: int | None = None) -> TextConfig:
        return TextConfig(n_layers or self.n_layers, self.hidden, self.n_heads, self.n_kv_heads, self.head_dim,
                          self.intermediate, vocab or self.vocab, self.rope_theta, self.rms_norm_eps)


QWEN3_ASR_0_6B = ModelSize("Qwen3-ASR-0.6B", hidden=1024, intermediate=3072)
QWEN3_ASR_1_7B = ModelSize("Qwen3-ASR-1.7B", hidden=2048, intermediate=6144)

# seeds of the synthetic inputs (one counter-based generator keyed by (seed, tensor name))
SEED_WEIGHTS = 20260101
SEED_INPUTS = 20260102
SEED_KV = 20260103
SEED_IDS = 20260104
SEED_LENGTHS = 20260105
STOP_IDS = (151645, 151643, 151645)   # im_end, endoftext, tokenizer eos (tools/qwen-asr-text-layer.cpp:395-399)


def synth_normal(n: int, seed: int, name: str, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib.qa_synth_fill_normal(fptr(out), n, seed, name.encode(), std)
    return out


def synth_ids(n: int, seed: int, name: str, lo: int, hi: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib.qa_synth_fill_ids(iptr(out), n, seed, name.encode(), lo, hi)
    return out


class Model:
    """Seeded synthetic Qwen3-ASR text model held in host memory (GGUF tensor names).

    bf16=True rounds every tensor to bf16 (kept as f32): the values of a checkpoint converted from
    the released bf16 weights (convert.py:386-387), for which the decoder streams bf16 copies."""

    def __init__(self, size: ModelSize, n_layers: int | None = None, seed: int = SEED_WEIGHTS,
                 vocab: int | None = None, bf16: bool = False):
        self.size = size
        self.cfg = size.config(n_layers, vocab)
        self.bf16 = bf16
        h = vp()
        check(lib.qa_model_synthetic(C.byref(self.cfg), seed, C.byref(h)))
        self.handle = h
        if bf16:
            check(lib.qa_model_round_bf16(h))

    def tensor(self, name: str) -> np.ndarray:
        n = i64()
        p = lib.qa_model_tensor(self.handle, name.encode(), C.byref(n))
        if not p:
            raise KeyError(name)
        return np.ctypeslib.as_array(p, shape=(n.value,))

    def weights(self):
        layers = (LayerWeights * self.cfg.n_layers)()
        w = ModelWeights()
        check(lib.qa_model_weights_view(self.handle, layers, self.cfg.n_layers, C.byref(w)))
        return layers, w

    def write_gguf(self, path: str):
        """Writes this model as a GGUF v3 checkpoint (qa_gguf_write_model)."""
        check(lib.qa_gguf_write_model(self.handle, os.fsencode(path)))

    def embed(self, ids) -> np.ndarray:
        e = self.tensor("text.token_embd.weight").reshape(self.cfg.vocab, self.cfg.hidden)
        return np.ascontiguousarray(e[np.asarray(ids, dtype=np.int64)])

    def close(self):
        if self.handle:
            lib.qa_model_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def build_asr_prompt(audio_tokens: int, system_text: str = "", language: str = "") -> str:
    """qwenasr_build_asr_prompt (tokenizer.cpp:529-549) through the C ABI."""
    n = sz()
    lib.qa_build_asr_prompt(audio_tokens, system_text.encode(), language.encode(), None, 0, C.byref(n))
    buf = C.create_string_buffer(n.value + 1)
    check(lib.qa_build_asr_prompt(audio_tokens, system_text.encode(), language.encode(), buf, n.value + 1, None))
    return buf.value.decode()


def wav_info(path: str) -> tuple[int, int]:
    """(sample frames, sample rate) of a WAV file as the reference's reader counts them."""
    n, rate = i64(), i32()
    check(lib.qa_wav_info(os.fsencode(path), C.byref(n), C.byref(rate)))
    return n.value, rate.value


def prompt_input(model: Model, audio_tokens: int, prompt_tokens: int) -> np.ndarray:
    """Decoder input [T][hidden]: audio-embedding rows N(0, 1) then embedded prompt ids U[0, vocab)."""
    h = model.cfg.hidden
    audio = synth_normal(audio_tokens * h, SEED_INPUTS, "audio_embeddings").reshape(audio_tokens, h)
    ids = synth_ids(prompt_tokens, SEED_IDS, "prompt_ids", 0, model.cfg.vocab - 1)
    return np.ascontiguousarray(np.concatenate([audio, model.embed(ids)], axis=0))


class Decoder:
    """C-ABI decoder: device weights + KV cache (qa_decoder_*)."""

    def __init__(self, model: Model, n_streams: int = 1, max_seq: int = 256, cache_type: int = QA_CACHE_F16):
        self.model = model
        self.cfg = model.cfg
        layers, w = model.weights()
        h = vp()
        check(lib.qa_decoder_create(C.byref(self.cfg), C.byref(w), n_streams, max_seq, cache_type, C.byref(h)))
        self.handle = h
        self.n_streams = n_streams
        self.max_seq = max_seq
        self.cache_type = cache_type

    def close(self):
        if self.handle:
            lib.qa_decoder_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def cur_len(self, stream: int = 0) -> int:
        v = i32()
        check(lib.qa_decoder_cur_len(self.handle, stream, C.byref(v)))
        return v.value

    @property
    def weights_bf16(self) -> bool:
        """True when the batch-1 GEMVs read bf16 copies of bf16-exact weights (qa_decoder_weights_bf16)."""
        return bool(lib.qa_decoder_weights_bf16(self.handle))

    def device_lens(self) -> np.ndarray:
        out = np.zeros(self.n_streams, dtype=np.int32)
        check(lib.qa_decoder_device_lens(self.handle, iptr(out)))
        return out

    def set_cur_len(self, stream: int, n: int):
        check(lib.qa_decoder_set_cur_len(self.handle, stream, n))

    def cache(self):
        lay = KvLayout()
        p = lib.qa_decoder_cache(self.handle, C.byref(lay))
        return p, lay

    def stream(self):
        return lib.qa_decoder_stream(self.handle)

    def forward(self, x: np.ndarray, n_past: int, want_logits: bool = True):
        x = np.ascontiguousarray(x, dtype=np.float32)
        t = x.shape[0]
        logits = np.empty(self.cfg.vocab, dtype=np.float32) if want_logits else None
        check(lib.qa_decoder_forward(self.handle, fptr(x), t, n_past, fptr(logits) if want_logits else None))
        return logits

    def generate(self, x: np.ndarray, max_new: int, stop_ids=STOP_IDS, margins: bool = False):
        x = np.ascontiguousarray(x, dtype=np.float32)
        ids = np.zeros(max(max_new, 1), dtype=np.int32)
        stops = np.asarray(stop_ids, dtype=np.int32)
        n_out, stopped, total = i32(), i32(), i32()
        marg = np.zeros(max(max_new, 1), dtype=np.float32) if margins else None
        check(lib.qa_decoder_generate(self.handle, fptr(x), x.shape[0], max_new, iptr(stops), len(stops), iptr(ids),
                                      C.byref(n_out), C.byref(stopped), C.byref(total),
                                      fptr(marg) if margins else None))
        out = dict(ids=ids[: n_out.value].tolist(), stopped=bool(stopped.value), total_tokens=total.value)
        if margins:
            out["margins"] = marg[: n_out.value].tolist()
        return out

    def decode_streams(self, first_ids: np.ndarray, n_steps: int) -> np.ndarray:
        first = np.ascontiguousarray(first_ids, dtype=np.int32)
        out = np.zeros((max(n_steps, 1), self.n_streams), dtype=np.int32)
        check(lib.qa_decoder_decode_streams(self.handle, iptr(first), n_steps, iptr(out)))
        return out[:n_steps]

    def set_persistent(self, enable: bool = True):
        """Batch-1 decode steps as one persistent launch for all layers (qa_decoder_set_persistent); raises
        QaError (QA_ERR_INVALID) where no persistent kernel covers the decoder's shapes."""
        check(lib.qa_decoder_set_persistent(self.handle, 1 if enable else 0))

    def fill_cache(self, stream: int, k: np.ndarray, v: np.ndarray, length: int):
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        check(lib.qa_decoder_fill_cache(self.handle, stream, fptr(k), fptr(v), length))

    def layer_forward(self, layer: int, x: np.ndarray, n_past: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty_like(x)
        check(lib.qa_decoder_layer_forward(self.handle, layer, fptr(x), x.shape[0], n_past, fptr(y)))
        return y

    def layer_forward_nocache(self, layer: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty_like(x)
        check(lib.qa_decoder_layer_forward_nocache(self.handle, layer, fptr(x), x.shape[0], fptr(y)))
        return y

    def prefill_nocache(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        logits = np.empty(self.cfg.vocab, dtype=np.float32)
        check(lib.qa_decoder_prefill_nocache(self.handle, fptr(x), x.shape[0], fptr(logits)))
        return logits

    # timing hooks (HIP events on the decoder's stream)
    def profile(self, enable: bool):
        check(lib.qa_decoder_profile_enable(self.handle, 1 if enable else 0))

    def profile_reset(self):
        check(lib.qa_decoder_profile_reset(self.handle))

    def profile_read(self, family: str):
        ms, n = C.c_double(), i64()
        check(lib.qa_decoder_profile_read(self.handle, family.encode(), C.byref(ms), C.byref(n)))
        return ms.value, n.value
