"""Synthetic models with bf16-exact weights (CPU).

qa_model_round_bf16 gives a synthetic model the values of a checkpoint converted from the released
bf16 weights (convert.py:386-387: each bf16 tensor is widened with tensor.float()).  Checked against
torch's own float32 -> bfloat16 conversion (round to nearest, ties to even)."""
import numpy as np
import torch


def torch_bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


def test_round_bf16_matches_torch(qa):
    plain = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=1, vocab=512)
    exact = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=1, vocab=512, bf16=True)
    names = ["text.blk.0.attn_q.weight", "text.blk.0.ffn_down.weight", "text.blk.0.attn_norm.weight",
             "text.token_embd.weight", "text.output.weight"]
    for name in names:
        a, b = plain.tensor(name), exact.tensor(name)
        np.testing.assert_array_equal(b.view(np.uint32), torch_bf16(a).view(np.uint32))
        assert not (b.view(np.uint32) & 0xffff).any()
    # tied LM head: one buffer, rounded once, still shared
    assert exact.tensor("text.output.weight").ctypes.data == exact.tensor("text.token_embd.weight").ctypes.data


def test_round_bf16_ties_and_specials(qa):
    """Halfway cases go to the even neighbour; exact values, zeros and infinities are unchanged."""
    m = qa.Model(qa.QWEN3_ASR_0_6B, n_layers=1, vocab=512)
    t = m.tensor("text.blk.0.attn_q.weight")
    bits = np.array([0x3f808000, 0x3f818000, 0x3f80ffff, 0x3f800001, 0x3f800000, 0x80000000, 0x7f800000,
                     0xff800000, 0x7f7fffff], np.uint32)
    t[: bits.size] = bits.view(np.float32)
    want = torch_bf16(bits.view(np.float32))
    qa.check(qa.lib.qa_model_round_bf16(m.handle))
    np.testing.assert_array_equal(t[: bits.size].view(np.uint32), want.view(np.uint32))
    # 1 + 2^-8 (halfway, even below) -> 1;  1 + 3 * 2^-8 (halfway, odd below) -> 1 + 2^-6
    assert t[0] == 1.0 and t[1] == np.float32(1.0 + 2.0 ** -6)
    assert np.isinf(t[8])                 # the largest finite f32 rounds up to infinity, as torch's
    # idempotent: a second rounding changes nothing
    before = t.copy()
    qa.check(qa.lib.qa_model_round_bf16(m.handle))
    np.testing.assert_array_equal(t.view(np.uint32), before.view(np.uint32))
