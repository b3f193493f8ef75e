"""Per-layer execution of a serving step over fixed fp32 state slots.

The caller of the memory block's ``packed`` in a serving step (the role of
``MemoryRuntime`` in runtime/executor.py:36-127).  What a step must do, and
what the tests pin:

* a step has two passes per memory layer, in order: the query pass (query
  samples whose session reads memory, ``memory_read[session]``) and the
  commit pass (every commit sample);
* a pass hands the block its samples' token rows and their slot states, and
  the block's residual rows go back to the same rows of the caller's
  ``output`` (rows of no pass stay zero);
* a commit's final state replaces its slot, and only after the block has
  read that slot, so a commit scans from, and reads, the state as it was
  before the step, and a query never sees a commit of the same step;
* every registered memory layer runs exactly once per step; lifecycle
  violations raise ``SessionError``, malformed buffers ``ValueError``, and a
  residual of the wrong shape or dtype ``RuntimeError``.

Slot state lives in ``pool.storage[layer]``, ``[slots, 1, H, K, V]`` fp32.
Each pass is described once (:class:`_Pass`: rows, lengths, slots) and then
executed either on a gathered copy of the slot states (``index_select`` /
``index_copy_`` on device index tensors) or, with ``slot_io=True`` and a
block that has ``packed_slots``, on the pool in place: the kernels read the
slots directly and write each commit's final state into its slot after every
read and initial state has been consumed.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from dataclasses import dataclass, field

import torch


class SessionError(RuntimeError):
    """A step lifecycle violation."""


@dataclass(frozen=True)
class MemoryRequest:
    """The part of a serving request the step reads."""

    rid: str
    session: str
    operation: str  # "query" or "commit"


@dataclass(frozen=True)
class Sample:
    """A request's token rows ``[start, stop)`` in the step."""

    request: MemoryRequest
    start: int
    stop: int

    @property
    def length(self) -> int:
        return self.stop - self.start


@dataclass(frozen=True)
class StepPlan:
    samples: tuple[Sample, ...]
    token_count: int


@dataclass(frozen=True)
class _Pass:
    """One call of the block: its samples' rows (a device index), lengths and slots."""

    commit: bool
    rows: torch.Tensor
    lengths: list[int]
    slots: list[int]


@dataclass
class _Step:
    plan: StepPlan
    slot_of: Mapping[str, int]
    memory_read: Mapping[str, bool]
    done: set = field(default_factory=set)  # memory layers executed in this step

    def passes(self, device) -> list[_Pass]:
        """The query pass (readable sessions only), then the commit pass; empty passes are dropped."""
        out = []
        for commit in (False, True):
            chosen = [s for s in self.plan.samples
                      if (s.request.operation == "commit") == commit
                      and (commit or self.memory_read[s.request.session])]
            if chosen:
                rows = torch.cat([torch.arange(s.start, s.stop) for s in chosen]).to(device)
                out.append(_Pass(commit, rows, [s.length for s in chosen],
                                 [self.slot_of[s.request.rid] for s in chosen]))
        return out


def _check_rows(hidden: torch.Tensor, output: torch.Tensor, token_count: int) -> None:
    """``hidden`` and ``output`` are distinct token-row matrices of one dtype
    and device covering the step's tokens."""
    if not (hidden.ndim == 2 and output.ndim == 2 and hidden.shape[0] == output.shape[0] >= token_count):
        raise ValueError(f"hidden {tuple(hidden.shape)} and residual {tuple(output.shape)} must be token-row "
                         f"matrices of equal length covering the step's {token_count} tokens")
    if (hidden.device, hidden.dtype) != (output.device, output.dtype):
        raise ValueError(f"residual ({output.dtype} on {output.device}) must match hidden "
                         f"({hidden.dtype} on {hidden.device})")
    shares = hidden.numel() > 0 and output.numel() > 0 and \
        hidden.untyped_storage().data_ptr() == output.untyped_storage().data_ptr()
    if shares:
        raise ValueError("the residual buffer shares storage with the hidden states")


class MemoryRuntime:
    """``pool.storage``: ``{layer: [slots, 1, H, K, V] fp32}``.  Per step,
    ``slot_of`` maps a request id to its slot (the session's published slot
    for a query, the transaction's candidate slot for a commit) and
    ``memory_read`` maps a session to whether its queries read memory."""

    def __init__(self, pool, *, slot_io: bool = False):
        self.pool = pool
        self.slot_io = slot_io
        self._step: _Step | None = None

    @property
    def plan(self) -> StepPlan | None:
        return None if self._step is None else self._step.plan

    def begin(self, plan: StepPlan, *, slot_of: Mapping[str, int], memory_read: Mapping[str, bool]) -> StepPlan:
        if self._step is not None:
            raise SessionError("begin() called while a step is still open")
        for s in plan.samples:
            if s.request.operation not in ("query", "commit"):
                raise ValueError(f"request {s.request.rid}: unknown operation {s.request.operation!r}")
            if not 0 <= s.start < s.stop <= plan.token_count:
                raise ValueError(f"request {s.request.rid}: token rows [{s.start}, {s.stop}) outside the step's "
                                 f"{plan.token_count} tokens")
        self._step = _Step(plan, slot_of, memory_read)
        return plan

    @torch.no_grad()
    def run_layer(self, layer: int, hidden: torch.Tensor, output: torch.Tensor, compute) -> torch.Tensor:
        """Run both passes of one memory layer and fill the caller's residual rows."""
        step = self._step
        if step is None:
            raise SessionError("run_layer() outside a step")
        if layer not in self.pool.storage:
            raise SessionError(f"layer {layer} has no memory state in the pool")
        if layer in step.done:
            raise SessionError(f"layer {layer} already ran in this step")
        _check_rows(hidden, output, step.plan.token_count)
        output.zero_()
        storage = self.pool.storage[layer]
        for p in step.passes(hidden.device):
            self._execute(p, hidden, output, storage, compute)
        step.done.add(layer)
        return output

    def _execute(self, p: _Pass, hidden, output, storage, compute) -> None:
        x = hidden.index_select(0, p.rows)
        if self.slot_io and hasattr(compute, "packed_slots"):
            residual = compute.packed_slots(x, storage, p.slots, p.slots, lengths=p.lengths, commit=p.commit)
            final, index = None, None
        else:
            index = torch.tensor(p.slots, dtype=torch.int64).to(hidden.device)
            # a gathered copy: the commit's initial state and read, so its final
            # state may replace the slot once the block has returned
            states = storage.index_select(0, index).view(len(p.slots), *storage.shape[2:])
            residual, final = compute.packed(x, states, lengths=p.lengths, commit=p.commit, write_states=states)
        if tuple(residual.shape) != (p.rows.numel(), output.shape[1]) or residual.dtype != output.dtype:
            raise RuntimeError(f"packed memory output invariant violated: residual {residual.dtype} "
                               f"{tuple(residual.shape)} for {p.rows.numel()} rows of {output.shape[1]}")
        output.index_copy_(0, p.rows, residual)
        if p.commit and final is not None:
            storage.index_copy_(0, index, final.unsqueeze(1))

    def finish(self, success: bool) -> None:
        """Close the step.  A successful step with samples must have run every
        memory layer of the pool; the step is closed either way.  (Advancing
        session lengths belongs to the session controller, the caller.)"""
        step, self._step = self._step, None
        if step is None:
            raise SessionError("finish() without an open step")
        missing = set(self.pool.storage.keys()) - step.done
        if success and step.plan.samples and missing:
            raise SessionError(f"step finished without running memory layers {sorted(missing)}")


def plan_of(requests: Sequence[tuple[MemoryRequest, int]]) -> StepPlan:
    """A step of consecutive samples from ``(request, token_count)`` pairs."""
    samples, offset = [], 0
    for request, n in requests:
        samples.append(Sample(request, offset, offset + int(n)))
        offset += int(n)
    return StepPlan(tuple(samples), offset)
