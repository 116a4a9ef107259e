import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "qwenasr.cpp_amd"), os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

# Logits of two f32 evaluations of the 28-layer decoder that differ only in summation order agree to
# LOGIT_ATOL (asserted by test_teacher_forced_logits_within_tolerance on the long-context config).
# A greedy pick can then differ only where the two top logits are closer than 2 * LOGIT_ATOL.
LOGIT_ATOL = 2e-3
TIE_EPS = 2 * LOGIT_ATOL

_GREEDY = pytest.StashKey[list]()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path through the C ABI)")
    config.addinivalue_line("markers", "slow: long CPU oracle runs")
    config.stash[_GREEDY] = []


# Accepted near-tie divergences per tie group over a session.  Only paths whose projections sum in
# another order than the default f32 kernels (the bf16-MFMA skinny GEMM and the bf16 prefill GEMM over the
# exact three-part split; the opt-in packed f32 multi-stream GEMMs) name a group; everything else, the
# BASELINE configs with their f32 weights on the default kernels included, must give identical ids.
TIE_CAP = {"config 3 bf16-exact": 1, "config 4 bf16-exact": 1, "config 4 packed f32": 1}


class GreedyRecorder:
    """Greedy-id comparisons of the session.  Ids must be identical.  The one exception is a comparison
    that names a tie group (TIE_CAP): there a first divergence at an oracle near-tie (top-2 margin <
    TIE_EPS) where the HIP path picked the oracle's runner-up is accepted, at most TIE_CAP[group] times
    per session; after it the two sequences feed different tokens and are not compared further.  Every
    comparison is recorded and the terminal summary prints the caps and the count per group."""

    def __init__(self, records: list):
        self.records = records

    def match(self, got, ref, margins, runner_up, what, tie_group=None):
        for i, (a, b) in enumerate(zip(got, ref)):
            if a != b:
                assert tie_group is not None, (f"{what}: ids differ at step {i} (HIP {a}, oracle {b}, oracle "
                                               f"margin {margins[i]:.3g}) on a path that allows no near-tie")
                assert margins[i] < TIE_EPS and a == runner_up[i], (what, i, a, b, margins[i], runner_up[i])
                used = sum(1 for r in self.records if r[6] == tie_group and r[2] is not None)
                assert used < TIE_CAP[tie_group], (f"{what}: near-tie cap of group '{tie_group}' "
                                                   f"({TIE_CAP[tie_group]}) exceeded at step {i}")
                self.records.append((what, len(ref), i, float(margins[i]), int(a), int(b), tie_group))
                return i
        assert len(got) == len(ref), (what, len(got), len(ref))
        self.records.append((what, len(ref), None, None, None, None, tie_group))
        return None


@pytest.fixture
def greedy(request):
    return GreedyRecorder(request.config.stash[_GREEDY])


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    recs = config.stash.get(_GREEDY, [])
    if not recs:
        return
    div = [r for r in recs if r[2] is not None]
    ids = sum(r[1] for r in recs)
    terminalreporter.write_line(
        f"greedy ids: {len(recs)} sequences ({ids} ids) compared, {len(recs) - len(div)} identical, "
        f"{len(div)} accepted near-tie divergence(s) (oracle top-2 margin < {TIE_EPS:g}, runner-up taken)")
    strict = [r for r in recs if r[6] is None]
    terminalreporter.write_line(f"  strict (no near-tie allowed): {len(strict)} sequences, all identical")
    for group, cap in TIE_CAP.items():
        n = sum(1 for r in recs if r[6] == group)
        used = sum(1 for r in div if r[6] == group)
        terminalreporter.write_line(f"  tie group '{group}': {n} sequences, {used} of cap {cap} near-ties used")
    for what, n, i, m, a, b, _ in div:
        terminalreporter.write_line(f"  near-tie: {what}: step {i} of {n}, oracle margin {m:.2e}, "
                                    f"HIP id {a} = oracle runner-up, oracle id {b}")


@pytest.fixture(scope="session")
def qa():
    import qwenasr_amd

    return qwenasr_amd


@pytest.fixture(scope="session")
def orc():
    import qa_oracle

    return qa_oracle
