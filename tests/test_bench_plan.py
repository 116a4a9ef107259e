"""bench.py's KV-cache capacity plan (CPU only).

Each decoder the bench creates must hold every position its legs write.  The legs are replayed here
against the decoder's capacity rule (qa_decoder_decode_streams refuses cur_len + n_steps > max_seq;
a cached forward refuses n_past + T > max_seq, text-decoder.cpp:1652-1656), for the driver's command
line (--steps 20 --warmup 5), the defaults, and edge cases.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402  (imports only the standard library at module level)


class Slot:
    """One stream's bookkeeping under the decoder's capacity rule."""

    def __init__(self, cap):
        self.cap, self.cur = cap, 0

    def forward(self, n_past, t):
        if n_past + t > self.cap:
            raise OverflowError(f"forward {n_past}+{t} > {self.cap}")
        self.cur = n_past + t

    def decode(self, n):
        if self.cur + n > self.cap:
            raise OverflowError(f"decode {self.cur}+{n} > {self.cap}")
        self.cur += n

    def attend_roofline(self):
        # attention_roofline appends at row cur and attends cur + 1 positions
        if self.cur + 1 > self.cap:
            raise OverflowError(f"roofline append at {self.cur} >= {self.cap}")


def replay(prompt, warmup, steps, profile_steps, bf16_steps, persistent_steps=32):
    plan = bench.capacity_plan(prompt, warmup, steps, profile_steps, bf16_steps, persistent_steps)
    main = Slot(plan["main"])
    for _ in range(3):                      # cold, steady-state and event-bracketed prefills
        main.forward(0, prompt)
    main.decode(warmup)
    main.decode(steps)
    main.decode(profile_steps)
    main.attend_roofline()
    if bf16_steps:
        side = Slot(plan["bf16_exact"])
        for _ in range(3):
            side.forward(0, prompt)
        side.decode(warmup)
        side.decode(bf16_steps)
    if persistent_steps:
        pers = Slot(plan["persistent"])
        pers.forward(0, prompt)
        pers.decode(warmup)
        pers.decode(persistent_steps)
    return plan


@pytest.mark.parametrize("warmup,steps", [(5, 20), (8, 256), (0, 1), (0, 0), (5, 4096), (64, 1)])
@pytest.mark.parametrize("bf16_steps", [0, 1, 64, 500])
def test_plan_holds_every_leg(warmup, steps, bf16_steps):
    # config 3's prompt (3913) and a short one
    for prompt in (3913, 156, 1):
        replay(prompt, warmup, steps, 8, bf16_steps)


def test_driver_command_line():
    """The driver runs `bench.py --gpus 1 --steps 20 --warmup 5`.  A side decoder given the main decoder's
    capacity overflows there (its 64 steps exceed the main run's 20 + 8); each decoder has its own."""
    plan = replay(3913, 5, 20, 8, 64)
    assert plan["main"] >= 3913 + 5 + 20 + 8 + 1
    assert plan["bf16_exact"] >= 3913 + 5 + 64
    assert plan["persistent"] >= 3913 + 5 + 32


def test_plan_is_not_oversized():
    # one spare row beyond the roofline's append: a cache sized from the plan has no slack to hide a bug
    plan = bench.capacity_plan(3913, 5, 20, 8, 64)
    with pytest.raises(OverflowError):
        s = Slot(plan["main"] - 2)
        s.forward(0, 3913)
        s.decode(5 + 20 + 8)
        s.attend_roofline()


def test_plan_rejects_bad_counts():
    with pytest.raises(ValueError):
        bench.capacity_plan(0, 5, 20, 8, 64)
    with pytest.raises(ValueError):
        bench.capacity_plan(3913, -1, 20, 8, 64)


def test_guarded_records_errors():
    out = {}

    def boom():
        raise RuntimeError("leg failed")

    assert bench.guarded(out, "leg", boom) == {"error": "RuntimeError: leg failed"}
    assert bench.guarded(out, "ok", lambda: {"v": 1}) == {"v": 1}
    assert out == {"leg": {"error": "RuntimeError: leg failed"}, "ok": {"v": 1}}


def test_parser_defaults_and_gpus_guard(capsys):
    """The default weights are the BASELINE draws as f32; --gpus above 1 exits with a message."""
    import subprocess

    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
    src = open(os.path.join(ROOT, "bench.py")).read()
    assert 'ap.add_argument("--weights", choices=["f32", "bf16-exact"], default="f32"' in src


def test_prefill_rooflines():
    """The prefill MFMA roofline objects: causal attention FLOPs at T = 3913 are BASELINE's 62.73 GFLOP per
    layer (4 x 16 x 128 x T (T + 1) / 2), the split-input GEMM does 3 x 2 T params per layer (50.33 M params
    per 1.7B layer), and the rate is FLOPs over the family's milliseconds."""
    import types

    cfg = types.SimpleNamespace(n_heads=16, head_dim=128, n_layers=28, hidden=2048, n_kv_heads=8, intermediate=6144)
    a = bench.prefill_attn_roofline(cfg, 3913, {"prefill_attn": 28 * 62.732214272e9 / 1e15 * 1e3})   # 1 PFLOP/s
    assert a["flop_per_layer"] == 62732214272
    assert abs(a["achieved"] - 1000.0) < 0.1 and a["bound"] == "mfma" and abs(a["frac"] - 0.4) < 1e-4
    params = (2048 + 2 * 1024) * 2048 + 2048 * 2048 + 2 * 6144 * 2048 + 2048 * 6144
    assert params == 50331648
    g = bench.prefill_gemm_roofline(cfg, 3913, {"projections": 30.0})
    assert g["flop_per_layer"] == 6 * 3913 * params
    assert abs(g["achieved"] - 28 * 6 * 3913 * params / 30e-3 / 1e12) < 0.1


def test_decode_weight_rooflines():
    """The batch-1 weight-stream objects: 1.7B layer projections are 50.33 M parameters (q|k|v 2048 x 4096, o 2048 x
    2048, gate|up 2 x 6144 x 2048, down 2048 x 6144), the LM head 151936 x 2048."""
    import qwenasr_amd as qa

    cfg = qa.QWEN3_ASR_1_7B.config()
    r = bench.decode_weight_rooflines(cfg, 4, {"projections": 1.0, "logits": 0.2})
    layer = 2048 * 4096 + 2048 * 2048 + 2 * 6144 * 2048 + 6144 * 2048
    assert layer == 50331648
    assert r["projections"]["bytes_per_token"] == 4 * 28 * layer
    assert abs(r["projections"]["achieved"] - 4 * 28 * layer / 1e-3 / 1e9) < 0.1
    assert r["lm_head"]["bytes_per_token"] == 4 * 151936 * 2048
    assert abs(r["lm_head"]["frac"] - 4 * 151936 * 2048 / 0.2e-3 / 1e9 / 8000) < 1e-4
    r16 = bench.decode_weight_rooflines(cfg, 2, {"projections": 1.0, "logits": 0.2})
    assert r16["projections"]["bytes_per_token"] * 2 == r["projections"]["bytes_per_token"]
