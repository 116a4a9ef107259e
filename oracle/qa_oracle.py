"""ctypes binding of the CPU oracle (libqa_oracle.so).

TEST INFRASTRUCTURE ONLY: the checker for the HIP path.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import this module; the product library never does.
See qa_oracle.h for what each function restates (file:line of andimarafioti/qwenasr.cpp).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ORACLE_DIR, "libqa_oracle.so")
if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built; run `make -C {ORACLE_DIR}`")
lib = C.CDLL(LIB_PATH)

i32, f32, sz = C.c_int32, C.c_float, C.c_size_t
fp, ip, u16p = C.POINTER(C.c_float), C.POINTER(C.c_int32), C.POINTER(C.c_uint16)


class Config(C.Structure):
    _fields_ = [("n_layers", i32), ("hidden", i32), ("n_heads", i32), ("n_kv_heads", i32), ("head_dim", i32),
                ("intermediate", i32), ("vocab", i32), ("rope_theta", f32), ("rms_norm_eps", f32)]


class Layer(C.Structure):
    _fields_ = [(n, fp) for n in ("attn_norm", "ffn_norm", "q", "k", "v", "o", "q_norm", "k_norm", "gate", "up",
                                  "down")]


class Model(C.Structure):
    _fields_ = [("cfg", Config), ("layers", C.POINTER(Layer)), ("token_embd", fp), ("output_norm", fp),
                ("output", fp)]


class Cache(C.Structure):
    _fields_ = [("dtype", i32), ("n_layers", i32), ("n_kv_heads", i32), ("head_dim", i32), ("max_seq", i32),
                ("cur_len", i32), ("k", C.c_void_p), ("v", C.c_void_p)]


def _sig(name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)


_sig("orc_f32_to_f16", C.c_uint16, f32)
_sig("orc_f16_to_f32", f32, C.c_uint16)
_sig("orc_f32_to_f16_array", None, fp, u16p, sz)
_sig("orc_f16_to_f32_array", None, u16p, fp, sz)
_sig("orc_rms_norm_row", None, fp, i32, fp, f32, fp)
_sig("orc_rope_rows", None, fp, i32, i32, i32, f32)
_sig("orc_slot_index", C.c_int64, i32, i32, i32, i32, i32)
_sig("orc_positions", None, i32, i32, ip)
_sig("orc_causal_mask", None, i32, i32, fp)
_sig("orc_linear", None, fp, i32, i32, fp, i32, fp)
_sig("orc_argmax", i32, fp, i32)
_sig("orc_set_threads", C.c_int, i32)
_sig("orc_qk_prep", None, fp, fp, i32, i32, i32, i32, fp, fp, i32, f32, f32)
_sig("orc_cache_write", None, C.POINTER(Cache), i32, fp, fp, i32, i32)
_sig("orc_cache_attention", None, C.POINTER(Cache), i32, fp, i32, i32, i32, f32, fp)
_sig("orc_causal_attention_f32", None, fp, fp, fp, i32, i32, i32, i32, f32, fp)
_sig("orc_layer_forward_cached", C.c_int, C.POINTER(Model), i32, fp, i32, i32, C.POINTER(Cache), fp)
_sig("orc_layer_forward_nocache", C.c_int, C.POINTER(Model), i32, fp, i32, fp)
_sig("orc_logits", C.c_int, C.POINTER(Model), fp, fp)
_sig("orc_forward_cached", C.c_int, C.POINTER(Model), fp, i32, i32, C.POINTER(Cache), fp)
_sig("orc_generate_cached", C.c_int, C.POINTER(Model), fp, i32, i32, ip, i32, C.POINTER(Cache), ip, ip, ip, ip, fp, ip)
_sig("orc_decode_steps", C.c_int, C.POINTER(Model), C.POINTER(Cache), i32, i32, ip, fp, ip)


def fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(fp)


def iptr(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(ip)


def set_threads(n: int) -> int:
    return lib.orc_set_threads(n)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib.orc_f32_to_f16_array(fptr(x.reshape(-1)), out.reshape(-1).ctypes.data_as(u16p), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib.orc_f16_to_f32_array(h.reshape(-1).ctypes.data_as(u16p), fptr(out.reshape(-1)), h.size)
    return out


def rms_norm_row(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty_like(x)
    lib.orc_rms_norm_row(fptr(x), x.size, fptr(w), eps, fptr(y))
    return y


def rope_rows(rows: np.ndarray, position: int, theta: float) -> np.ndarray:
    r = np.array(rows, dtype=np.float32, copy=True, order="C")
    n_heads, d = r.shape
    lib.orc_rope_rows(fptr(r), position, n_heads, d, theta)
    return r


def linear(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, in_dim = x.shape
    out_dim = w.shape[0]
    y = np.empty((rows, out_dim), dtype=np.float32)
    lib.orc_linear(fptr(x), rows, in_dim, fptr(w), out_dim, fptr(y))
    return y


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return int(lib.orc_argmax(fptr(v), v.size))


class OracleCache:
    """One stream's KV cache: K and V each [n_layers][n_kv_heads][max_seq][head_dim] (f32 or f16 bits)."""

    def __init__(self, n_layers: int, n_kv_heads: int, head_dim: int, max_seq: int, f16: bool):
        dt = np.uint16 if f16 else np.float32
        shape = (n_layers, n_kv_heads, max_seq, head_dim)
        self.k = np.zeros(shape, dtype=dt)
        self.v = np.zeros(shape, dtype=dt)
        self.f16 = f16
        self.c = Cache(1 if f16 else 0, n_layers, n_kv_heads, head_dim, max_seq, 0,
                       self.k.ctypes.data_as(C.c_void_p), self.v.ctypes.data_as(C.c_void_p))

    @property
    def cur_len(self) -> int:
        return self.c.cur_len

    @cur_len.setter
    def cur_len(self, n: int):
        self.c.cur_len = n

    def k_f32(self) -> np.ndarray:
        return f16_bits_to_f32(self.k) if self.f16 else self.k

    def v_f32(self) -> np.ndarray:
        return f16_bits_to_f32(self.v) if self.f16 else self.v

    def fill(self, k: np.ndarray, v: np.ndarray, length: int):
        """k, v: f32 [n_layers][n_kv_heads][length][head_dim] written to rows [0, length)."""
        if self.f16:
            self.k[:, :, :length] = f32_to_f16_bits(k)
            self.v[:, :, :length] = f32_to_f16_bits(v)
        else:
            self.k[:, :, :length] = k
            self.v[:, :, :length] = v
        self.cur_len = length


class OracleModel:
    """orc_model over host weight arrays (kept alive by this object)."""

    def __init__(self, cfg: dict, layers: list[dict], token_embd, output_norm, output):
        self._keep = []
        c = Config(cfg["n_layers"], cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"],
                   cfg["intermediate"], cfg["vocab"], cfg["rope_theta"], cfg["rms_norm_eps"])
        arr = (Layer * cfg["n_layers"])()
        for i, lw in enumerate(layers):
            for name, _ in Layer._fields_:
                a = np.ascontiguousarray(lw[name], dtype=np.float32)
                self._keep.append(a)
                setattr(arr[i], name, fptr(a))
        self._keep.append(arr)
        ptrs = []
        for a in (token_embd, output_norm, output):
            if a is None:
                ptrs.append(None)
            else:
                a = np.ascontiguousarray(a, dtype=np.float32)
                self._keep.append(a)
                ptrs.append(fptr(a))
        self.m = Model(c, arr, *ptrs)
        self.cfg = cfg

    @classmethod
    def from_product_model(cls, model) -> "OracleModel":
        """Wrap the host tensors of a qwenasr_amd.Model (same bits the GPU receives; no copy)."""
        c = model.cfg
        cfg = dict(n_layers=c.n_layers, hidden=c.hidden, n_heads=c.n_heads, n_kv_heads=c.n_kv_heads,
                   head_dim=c.head_dim, intermediate=c.intermediate, vocab=c.vocab, rope_theta=c.rope_theta,
                   rms_norm_eps=c.rms_norm_eps)
        names = dict(attn_norm="attn_norm", ffn_norm="ffn_norm", q="attn_q", k="attn_k", v="attn_v",
                     o="attn_output", q_norm="attn_q_norm", k_norm="attn_k_norm", gate="ffn_gate", up="ffn_up",
                     down="ffn_down")
        layers = [{k: model.tensor(f"text.blk.{l}.{n}.weight") for k, n in names.items()} for l in range(c.n_layers)]
        return cls(cfg, layers, model.tensor("text.token_embd.weight"), model.tensor("text.output_norm.weight"),
                   model.tensor("text.output.weight"))

    def cache(self, max_seq: int, f16: bool) -> OracleCache:
        c = self.cfg
        return OracleCache(c["n_layers"], c["n_kv_heads"], c["head_dim"], max_seq, f16)

    def layer_forward_cached(self, layer: int, x: np.ndarray, n_past: int, cache: OracleCache) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty_like(x)
        rc = lib.orc_layer_forward_cached(C.byref(self.m), layer, fptr(x), x.shape[0], n_past, C.byref(cache.c),
                                          fptr(y))
        assert rc == 0, rc
        cache.cur_len = n_past + x.shape[0]
        return y

    def layer_forward_nocache(self, layer: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty_like(x)
        assert lib.orc_layer_forward_nocache(C.byref(self.m), layer, fptr(x), x.shape[0], fptr(y)) == 0
        return y

    def forward_cached(self, x: np.ndarray, n_past: int, cache: OracleCache) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        logits = np.empty(self.cfg["vocab"], dtype=np.float32)
        rc = lib.orc_forward_cached(C.byref(self.m), fptr(x), x.shape[0], n_past, C.byref(cache.c), fptr(logits))
        assert rc == 0, rc
        return logits

    def prefill_nocache(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        a = x
        for l in range(self.cfg["n_layers"]):
            a = self.layer_forward_nocache(l, a)
        logits = np.empty(self.cfg["vocab"], dtype=np.float32)
        lib.orc_logits(C.byref(self.m), fptr(np.ascontiguousarray(a[-1])), fptr(logits))
        return logits

    def generate(self, x: np.ndarray, max_new: int, stop_ids, cache: OracleCache):
        x = np.ascontiguousarray(x, dtype=np.float32)
        ids = np.zeros(max(max_new, 1), dtype=np.int32)
        marg = np.zeros(max(max_new, 1), dtype=np.float32)
        second = np.zeros(max(max_new, 1), dtype=np.int32)
        stops = np.asarray(stop_ids, dtype=np.int32)
        n_out, stopped, total = i32(), i32(), i32()
        rc = lib.orc_generate_cached(C.byref(self.m), fptr(x), x.shape[0], max_new, iptr(stops), len(stops),
                                     C.byref(cache.c), iptr(ids), C.byref(n_out), C.byref(stopped), C.byref(total),
                                     fptr(marg), iptr(second))
        n = n_out.value
        return dict(rc=rc, ids=ids[:n].tolist(), stopped=bool(stopped.value), total_tokens=total.value,
                    margins=marg[:n].tolist(), runner_up=second[:n].tolist(), cur_len=cache.cur_len)

    def decode_steps(self, cache: OracleCache, first_id: int, n_steps: int):
        """-> (ids, margins, runner_up) of n_steps greedy steps from first_id at cache.cur_len."""
        ids = np.zeros(n_steps, dtype=np.int32)
        marg = np.zeros(n_steps, dtype=np.float32)
        second = np.zeros(n_steps, dtype=np.int32)
        rc = lib.orc_decode_steps(C.byref(self.m), C.byref(cache.c), first_id, n_steps, iptr(ids), fptr(marg),
                                  iptr(second))
        assert rc == 0, rc
        return ids.tolist(), marg.tolist(), second.tolist()


def cache_attention(k: np.ndarray, v: np.ndarray, q: np.ndarray, n_past: int, f16: bool, library=None) -> np.ndarray:
    """Attention of T queries q [T][H][d] (positions n_past..) over one layer's cache rows.
    k, v: f32 values [n_kv][L][d] with L = n_past + T (rounded to f16 first when f16).
    `library` runs another build of qa_oracle.c (the planted-mistake builds of the oracle's tests)."""
    n_kv, L, d = k.shape
    T, H, _ = q.shape
    assert L == n_past + T
    cache = OracleCache(1, n_kv, d, L, f16)
    cache.fill(k[None], v[None], L)
    out = np.empty((T, H, d), dtype=np.float32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    (library or lib).orc_cache_attention(C.byref(cache.c), 0, fptr(q), n_past, T, H, 1.0 / np.sqrt(np.float32(d)),
                                         fptr(out))
    return out


def load_build(path: str):
    """ctypes handle of another build of qa_oracle.c with the attention entry point typed."""
    other = C.CDLL(path)
    f = other.orc_cache_attention
    f.restype = None
    f.argtypes = [C.POINTER(Cache), i32, fp, i32, i32, i32, f32, fp]
    return other


def causal_attention_f32(q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
    """q [T][H][d], k/v [T][n_kv][d] f32 -> [T][H][d] (non-cached causal attention)."""
    T, H, d = q.shape
    n_kv = k.shape[1]
    out = np.empty((T, H, d), dtype=np.float32)
    lib.orc_causal_attention_f32(fptr(np.ascontiguousarray(q, dtype=np.float32)),
                                 fptr(np.ascontiguousarray(k, dtype=np.float32)),
                                 fptr(np.ascontiguousarray(v, dtype=np.float32)), T, H, n_kv, d,
                                 1.0 / np.sqrt(np.float32(d)), fptr(out))
    return out


def qk_prep(q: np.ndarray, k: np.ndarray, q_norm_w, k_norm_w, pos0: int, theta: float, eps: float):
    """q [T][H][d], k [T][n_kv][d] -> normed + roped copies."""
    q = np.array(q, dtype=np.float32, copy=True, order="C")
    k = np.array(k, dtype=np.float32, copy=True, order="C")
    T, H, d = q.shape
    lib.orc_qk_prep(fptr(q), fptr(k), T, H, k.shape[1], d, fptr(np.ascontiguousarray(q_norm_w, dtype=np.float32)),
                    fptr(np.ascontiguousarray(k_norm_w, dtype=np.float32)), pos0, theta, eps)
    return q, k
