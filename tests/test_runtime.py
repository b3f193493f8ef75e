"""The serving caller of the memory block (runtime/executor.py:36-127) on the
CPU, with a fake state pool and a fake block whose ``packed`` records what it
was given: pass order, memory_read gating, which state each sample reads,
the residual scatter, and the commit writing ``final`` into its slot."""

import pytest
import torch

from memt_gdn2.runtime import MemoryRequest, MemoryRuntime, SessionError, StepPlan, plan_of

H, K, V, HID = 2, 4, 4, 8


class FakePool:
    def __init__(self, layers=(0, 3), slots=6, seed=0):
        g = torch.Generator().manual_seed(seed)
        self.storage = {layer: torch.randn(slots, 1, H, K, V, generator=g) for layer in layers}


class RecordingBlock:
    """``packed`` returns residual row t = hidden[t] * (1 + sum of its sample's
    state) and, for commits, final = state * 2 + 1; it records every call."""

    def __init__(self, residual_dtype=None, residual_rows=None):
        self.calls = []
        self.residual_dtype = residual_dtype
        self.residual_rows = residual_rows

    def packed(self, hidden_states, read_states, *, lengths, commit, write_states):
        assert read_states is write_states
        self.calls.append(dict(commit=commit, lengths=list(lengths), hidden=hidden_states.clone(),
                               states=read_states.clone()))
        sums = read_states.sum(dim=(1, 2, 3))
        per_row = torch.repeat_interleave(sums, torch.tensor(lengths))
        residual = hidden_states * (1 + per_row[:, None])
        if self.residual_dtype is not None:
            residual = residual.to(self.residual_dtype)
        if self.residual_rows is not None:
            residual = residual[: self.residual_rows]
        final = read_states * 2 + 1 if commit else None
        return residual, final


def _step(specs):
    """specs: (rid, session, operation, tokens)."""
    return plan_of([(MemoryRequest(rid, session, op), n) for rid, session, op, n in specs])


def _run(plan, slot_of, memory_read, block, pool=None, layers=None):
    pool = pool or FakePool()
    rt = MemoryRuntime(pool)
    rt.begin(plan, slot_of=slot_of, memory_read=memory_read)
    hidden = torch.randn(plan.token_count + 2, HID, generator=torch.Generator().manual_seed(1))
    outputs = {}
    for layer in (layers if layers is not None else pool.storage):
        out = torch.full_like(hidden, 7.0)
        rt.run_layer(layer, hidden, out, block)
        outputs[layer] = out
    rt.finish(True)
    return pool, hidden, outputs


def test_queries_run_before_commits_and_read_pre_commit_state():
    # the commit comes first in token order, the query of another session second
    plan = _step([("c1", "s1", "commit", 3), ("q1", "s2", "query", 2)])
    slot_of = {"c1": 4, "q1": 1}
    pool = FakePool(layers=(0,))
    before = pool.storage[0].clone()
    block = RecordingBlock()
    pool, hidden, out = _run(plan, slot_of, {"s1": True, "s2": True}, block, pool)
    assert [c["commit"] for c in block.calls] == [False, True]
    q_call, c_call = block.calls
    assert q_call["lengths"] == [2] and c_call["lengths"] == [3]
    assert torch.equal(q_call["states"], before[1:2].view(1, H, K, V))
    assert torch.equal(c_call["states"], before[4:5].view(1, H, K, V))
    assert torch.equal(q_call["hidden"], hidden[3:5]) and torch.equal(c_call["hidden"], hidden[0:3])


def test_commit_final_replaces_its_slot_only():
    plan = _step([("c1", "s1", "commit", 3), ("c2", "s2", "commit", 5), ("q", "s3", "query", 1)])
    slot_of = {"c1": 2, "c2": 5, "q": 0}
    pool = FakePool()
    before = {layer: t.clone() for layer, t in pool.storage.items()}
    _run(plan, slot_of, {"s1": True, "s2": True, "s3": True}, RecordingBlock(), pool)
    for layer, t in pool.storage.items():
        for slot in range(t.shape[0]):
            want = before[layer][slot] * 2 + 1 if slot in (2, 5) else before[layer][slot]
            assert torch.equal(t[slot], want), (layer, slot)


def test_residual_rows_scattered_and_rest_zeroed():
    plan = _step([("q1", "s1", "query", 2), ("c1", "s2", "commit", 3), ("q2", "s3", "query", 1)])
    slot_of = {"q1": 0, "c1": 3, "q2": 1}
    pool = FakePool(layers=(0,))
    before = pool.storage[0].clone()
    pool, hidden, out = _run(plan, slot_of, {"s1": True, "s2": True, "s3": True}, RecordingBlock(), pool)
    out = out[0]
    for (a, b), slot in (((0, 2), 0), ((2, 5), 3), ((5, 6), 1)):
        scale = 1 + before[slot].sum()
        assert torch.allclose(out[a:b], hidden[a:b] * scale)
    assert torch.equal(out[6:], torch.zeros_like(out[6:]))  # rows past the samples: zero, not 7


def test_memory_read_gates_queries_not_commits():
    plan = _step([("q1", "s1", "query", 2), ("c1", "s1b", "commit", 2), ("q2", "s2", "query", 2)])
    slot_of = {"q1": 0, "c1": 3, "q2": 1}
    block = RecordingBlock()
    pool, hidden, out = _run(plan, slot_of, {"s1": False, "s1b": False, "s2": True}, block,
                             FakePool(layers=(0,)))
    assert [(c["commit"], c["lengths"]) for c in block.calls] == [(False, [2]), (True, [2])]
    assert torch.equal(block.calls[0]["hidden"], hidden[4:6])
    assert torch.equal(out[0][0:2], torch.zeros(2, HID))


def test_no_samples_leaves_output_zero_and_no_calls():
    block = RecordingBlock()
    pool, hidden, out = _run(StepPlan((), 0), {}, {}, block, FakePool(layers=(0,)))
    assert block.calls == [] and torch.equal(out[0], torch.zeros_like(out[0]))


@pytest.mark.parametrize("bad", [dict(residual_dtype=torch.float64), dict(residual_rows=1)])
def test_residual_invariant_raises_runtime_error(bad):
    plan = _step([("q1", "s1", "query", 2)])
    rt = MemoryRuntime(FakePool(layers=(0,)))
    rt.begin(plan, slot_of={"q1": 0}, memory_read={"s1": True})
    hidden = torch.randn(2, HID)
    with pytest.raises(RuntimeError, match="invariant"):
        rt.run_layer(0, hidden, torch.empty_like(hidden), RecordingBlock(**bad))


def test_lifecycle_errors():
    pool = FakePool(layers=(0, 1))
    rt = MemoryRuntime(pool)
    plan = _step([("q1", "s1", "query", 2)])
    hidden = torch.randn(2, HID)
    with pytest.raises(SessionError):
        rt.run_layer(0, hidden, torch.empty_like(hidden), RecordingBlock())  # no step
    rt.begin(plan, slot_of={"q1": 0}, memory_read={"s1": True})
    with pytest.raises(SessionError):
        rt.begin(plan, slot_of={"q1": 0}, memory_read={"s1": True})
    with pytest.raises(ValueError):
        rt.run_layer(0, hidden, hidden, RecordingBlock())  # aliasing residual
    with pytest.raises(ValueError):
        rt.run_layer(0, hidden, torch.empty(2, HID, dtype=torch.float64), RecordingBlock())
    with pytest.raises(ValueError):
        rt.run_layer(0, hidden[:1], torch.empty(1, HID), RecordingBlock())  # fewer rows than the step
    rt.run_layer(0, hidden, torch.empty_like(hidden), RecordingBlock())
    with pytest.raises(SessionError):
        rt.run_layer(0, hidden, torch.empty_like(hidden), RecordingBlock())  # layer twice
    with pytest.raises(SessionError):
        rt.run_layer(7, hidden, torch.empty_like(hidden), RecordingBlock())  # unknown layer
    with pytest.raises(SessionError):
        rt.finish(True)  # layer 1 never ran
    assert rt.plan is None
    rt.begin(plan, slot_of={"q1": 0}, memory_read={"s1": True})
    rt.finish(False)  # a failed step need not run every layer
    with pytest.raises(SessionError):
        rt.finish(True)


def test_invalid_plans_rejected():
    rt = MemoryRuntime(FakePool(layers=(0,)))
    with pytest.raises(ValueError):
        rt.begin(StepPlan((plan_of([(MemoryRequest("a", "s", "publish"), 2)]).samples), 2), slot_of={},
                 memory_read={})
    bad = plan_of([(MemoryRequest("a", "s", "query"), 2)])
    with pytest.raises(ValueError):
        rt.begin(StepPlan(bad.samples, 1), slot_of={"a": 0}, memory_read={"s": True})
