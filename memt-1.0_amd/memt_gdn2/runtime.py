"""Per-layer execution of a serving step over fixed fp32 state slots.

Counterpart of ``MemoryRuntime.run_layer`` / ``_run_prepared``
(runtime/executor.py:36-110), the caller of the memory block's ``packed``.
Per memory layer and step:

1. query samples run first, and only for sessions whose memory is readable
   (``memory_read[session]``); commit samples run second, always;
2. each pass gathers its samples' token rows and their slot states, calls
   ``compute.packed(rows, states, lengths=..., commit=..., write_states=states)``;
3. the residual rows are scattered back into the caller's ``output``; a
   commit's ``final`` state replaces its transaction slot.

The gathered states are a copy, so a commit reads and scans from the slot's
state as it was before the step, and queries (run first) never see a commit
of the same step.  Slot state lives in ``pool.storage[layer]``, a tensor
``[slots, 1, H, K, V]`` fp32.

The gather is ``index_select`` on a device index tensor and the scatter
``index_copy_``, one kernel each, where the reference concatenates per-slot
views (executor.py:86-91).  The values moved are the same.  With
``slot_io=True`` and a block that has ``packed_slots``, neither happens: the
kernels read the slots in place and write each commit's final state into its
slot (the read and every initial state are consumed before any final state
is stored).
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from dataclasses import dataclass

import torch


class SessionError(RuntimeError):
    """A step lifecycle violation (protocol.SessionError in the reference)."""


@dataclass(frozen=True)
class MemoryRequest:
    """What the executor reads of a request (protocol.MemoryRequest)."""

    rid: str
    session: str
    operation: str  # "query" or "commit"


@dataclass(frozen=True)
class Sample:
    """A request's token rows ``[start, stop)`` in the step (runtime/plan.py:8-14)."""

    request: MemoryRequest
    start: int
    stop: int


@dataclass(frozen=True)
class StepPlan:
    samples: tuple[Sample, ...]
    token_count: int


class MemoryRuntime:
    """``pool.storage``: ``{layer: [slots, 1, H, K, V] fp32}``.  ``slot_of``
    maps a request id to its slot (the session's published slot for a query,
    the transaction's candidate slot for a commit); ``memory_read`` maps a
    session to whether its queries read memory."""

    def __init__(self, pool, *, slot_io: bool = False):
        self.pool = pool
        self.slot_io = slot_io
        self.plan: StepPlan | None = None
        self._layers: set[int] = set()
        self.slot_of: Mapping[str, int] = {}
        self.memory_read: Mapping[str, bool] = {}

    def begin(self, plan: StepPlan, *, slot_of: Mapping[str, int], memory_read: Mapping[str, bool]) -> StepPlan:
        if self.plan is not None:
            raise SessionError("Previous step has not finished")
        for sample in plan.samples:
            if sample.request.operation not in ("query", "commit"):
                raise ValueError(f"unknown operation {sample.request.operation!r}")
            if not 0 <= sample.start < sample.stop <= plan.token_count:
                raise ValueError("Invalid request token span")
        self.plan = plan
        self.slot_of = slot_of
        self.memory_read = memory_read
        return plan

    @torch.no_grad()
    def run_layer(self, layer: int, hidden: torch.Tensor, output: torch.Tensor, compute) -> torch.Tensor:
        """Execute the step's samples for one memory layer and fill the
        caller-owned residual rows (executor.py:36-62)."""
        if self.plan is None or layer in self._layers or layer not in self.pool.storage:
            raise SessionError("Each registered memory layer must run once per step")
        if hidden.ndim != 2 or output.ndim != 2 or len(hidden) != len(output) or len(hidden) < self.plan.token_count:
            raise ValueError("Expected token-row hidden and residual buffers")
        if hidden.device != output.device or hidden.dtype != output.dtype:
            raise ValueError("Residual buffer must match hidden dtype and device")
        if hidden.numel() and output.numel() and \
                hidden.untyped_storage().data_ptr() == output.untyped_storage().data_ptr():
            raise ValueError("Residual buffer must not alias hidden states")
        output.zero_()
        self._run_prepared(layer, hidden, output, compute)
        self._layers.add(layer)
        return output

    def _pass_samples(self, commit: bool) -> list[Sample]:
        return [
            s for s in self.plan.samples
            if (s.request.operation == "commit") == commit and (commit or self.memory_read[s.request.session])
        ]

    def _run_prepared(self, layer: int, hidden: torch.Tensor, output: torch.Tensor, compute) -> None:
        storage = self.pool.storage[layer]
        dev = hidden.device
        for commit in (False, True):
            samples = self._pass_samples(commit)
            if not samples:
                continue
            rows = torch.cat([torch.arange(s.start, s.stop) for s in samples]).to(dev)
            lengths = [s.stop - s.start for s in samples]
            slot_list = [self.slot_of[s.request.rid] for s in samples]
            if self.slot_io and hasattr(compute, "packed_slots"):
                residual = compute.packed_slots(hidden.index_select(0, rows), storage, slot_list, slot_list,
                                                lengths=lengths, commit=commit)
                final = None
            else:
                slots = torch.tensor(slot_list, dtype=torch.int64).to(dev)
                # a copy: the scan's initial state, so `final` may replace the slot afterwards
                states = storage.index_select(0, slots).view(len(samples), *storage.shape[2:])
                residual, final = compute.packed(hidden.index_select(0, rows), states, lengths=lengths,
                                                 commit=commit, write_states=states)
            if residual.shape != (len(rows), output.shape[1]) or residual.dtype != output.dtype:
                raise RuntimeError("Packed memory output invariant violated")
            output.index_copy_(0, rows, residual)
            if commit and final is not None:
                storage.index_copy_(0, slots, final.unsqueeze(1))

    def finish(self, success: bool) -> None:
        """End the step; on success every registered layer must have run
        (executor.py:112-127).  Advancing session lengths is the session
        controller's business and stays with the caller."""
        if self.plan is None:
            raise SessionError("No active memory step")
        try:
            if success and self.plan.samples and self._layers != set(self.pool.storage.keys()):
                raise SessionError("Not all memory layers executed")
        finally:
            self.plan = None
            self._layers.clear()


def plan_of(requests: Sequence[tuple[MemoryRequest, int]]) -> StepPlan:
    """A step of consecutive samples from ``(request, token_count)`` pairs."""
    samples, offset = [], 0
    for request, n in requests:
        samples.append(Sample(request, offset, offset + int(n)))
        offset += int(n)
    return StepPlan(tuple(samples), offset)
