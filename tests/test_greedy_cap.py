"""The greedy-id comparison rule of the GPU tests (CPU only): identical ids, except a capped number of
oracle near-ties on the paths that name a tie group."""
import pytest

from conftest import TIE_CAP, TIE_EPS, GreedyRecorder


def test_identical_ids_pass_everywhere():
    g = GreedyRecorder([])
    assert g.match([1, 2, 3], [1, 2, 3], [1.0] * 3, [9] * 3, "strict") is None
    assert g.match([1, 2, 3], [1, 2, 3], [1.0] * 3, [9] * 3, "grouped", tie_group="config 4 bf16-exact") is None


def test_strict_path_fails_even_at_a_near_tie():
    g = GreedyRecorder([])
    with pytest.raises(AssertionError, match="allows no near-tie"):
        g.match([1, 7, 3], [1, 2, 3], [1.0, TIE_EPS / 100, 1.0], [9, 7, 9], "config 3")


def test_tie_group_accepts_runner_up_at_near_tie_up_to_cap():
    g = GreedyRecorder([])
    group = "config 4 bf16-exact"
    assert g.match([1, 7, 5], [1, 2, 3], [1.0, 1e-5, 1.0], [9, 7, 9], "stream 0", tie_group=group) == 1
    for _ in range(TIE_CAP[group] - 1):
        g.match([7], [2], [1e-5], [7], "stream n", tie_group=group)
    with pytest.raises(AssertionError, match="cap"):
        g.match([7], [2], [1e-5], [7], "stream 31", tie_group=group)


def test_tie_group_rejects_wide_margins_and_other_ids():
    g = GreedyRecorder([])
    group = "config 3 bf16-exact"
    with pytest.raises(AssertionError):
        g.match([7], [2], [TIE_EPS * 2], [7], "wide margin", tie_group=group)
    with pytest.raises(AssertionError):
        g.match([8], [2], [1e-5], [7], "not the runner-up", tie_group=group)


def test_length_mismatch_fails():
    g = GreedyRecorder([])
    with pytest.raises(AssertionError):
        g.match([1, 2], [1, 2, 3], [1.0] * 3, [9] * 3, "short")
