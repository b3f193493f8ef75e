"""Memory blocks of the Nano and Flash models on the HIP operators.

``QwenMemoryBlock`` keeps the reference block's parameter names and shapes
(models/qwen/layer.py:34-69), so a checkpoint's state dict loads unchanged,
and its ``packed`` entry (models/qwen/layer.py:99-152), the one call the
serving runtime makes per memory layer.  The dense projections stay torch
GEMMs (hipBLASLt).  Everything after them runs in this package's kernels:

* decode batches (every query sample one token long): one fused kernel,
  ``l2norm(q)``, the read of each sample's state and ``MemTRMSNormGated``;
* other query samples: ``l2norm`` -> ``memt_gdn2_read_fwd`` -> ``MemTRMSNormGated``;
* commit samples: the update with the gate and q/k prologue inside its WY
  kernel (``fused_prologue=True``, the default), or one prologue kernel
  (gates, ``l2norm(q)``, ``sqrt_b * l2norm(k)``) then ``token_memory_packed``;
  then ``MemTRMSNormGated``.

``DeepSeekMemoryBlock`` does the same for the Flash model
(models/deepseek/layer.py:46-183): grouped low-rank Q/K/V and gate
projections in torch, then the update with the prologue inside its WY kernel
(or the prologue kernel and ``token_memory_packed_flash``), or the snapshot
read for queries, and the gated RMSNorm, at d = 512.
"""

from __future__ import annotations

from itertools import accumulate

import torch
from torch import nn
from torch.nn import functional as F

from .layout import WY_TILE_TOKENS, build_chunk_plan, validate_packed_inputs
from .norm import MemTRMSNormGated
from .ops import (l2norm, memory_prologue, memt_gdn2_read_fwd, read_slots, readout_decode, snapshot_read,
                  token_memory_packed, token_memory_packed_flash, token_memory_packed_fused,
                  token_memory_packed_fused_slots, token_memory_packed_slots)


class QwenMemoryBlock(nn.Module):
    """``memory_config`` needs ``hidden_size``, ``num_heads``, ``head_dim``,
    ``chunk_tokens``, ``rms_norm_eps`` and ``output_gate_softcap``."""

    def __init__(self, memory_config, *, device=None, fused_prologue: bool = True):
        super().__init__()
        self.fused_prologue = fused_prologue
        hidden_size = memory_config.hidden_size
        num_heads = memory_config.num_heads
        head_dim = memory_config.head_dim
        self.chunk_tokens = memory_config.chunk_tokens
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.value_dim = num_heads * head_dim
        self.read_scale = head_dim ** -0.5
        width = num_heads * head_dim
        # in_proj rows: q, k, v, erase, write (H*D each), decay latent, output-gate latent (D each)
        self.qkv_rows = (width,) * 3
        self.gate_rows = (width, width, head_dim, head_dim)
        self.qkv_width = 3 * width
        self.write_gate_rows = self.gate_rows[:-1]
        self._write_gate_slice = slice(self.qkv_width, self.qkv_width + sum(self.write_gate_rows))
        self.in_proj = nn.Linear(hidden_size, self.qkv_width + sum(self.gate_rows), bias=False)
        self.f_down = nn.Linear(head_dim, width, bias=False)
        self.g_down = nn.Linear(head_dim, width, bias=False)
        self.decay_scale_log = nn.Parameter(torch.zeros(num_heads))
        self.decay_bias = nn.Parameter(torch.zeros(width))
        self.o_norm = MemTRMSNormGated(head_dim, eps=memory_config.rms_norm_eps,
                                       output_gate_softcap_limit=memory_config.output_gate_softcap)
        self.to(device=device, dtype=torch.bfloat16)
        self.eval()

    @torch.no_grad()
    def packed(self, hidden_states, read_states, *, lengths, commit, write_states):
        """``(residual [T, H*D] bf16, next_state [N,H,D,D] fp32 | None)``.

        Query samples (``commit=False``) read ``read_states[n]`` for every
        token of sample ``n``.  Commit samples also scan their tokens from
        ``write_states[n]``; their read still sees ``read_states[n]``, the
        state before the commit."""
        validate_packed_inputs(self, hidden_states, read_states, write_states, lengths)
        T, H, D = len(hidden_states), self.num_heads, self.head_dim
        hidden_batch = hidden_states.unsqueeze(0)
        weight = self.in_proj.weight
        q, k, v = F.linear(hidden_batch, weight[: self.qkv_width]).split(self.qkv_rows, dim=-1)
        output_gate = self.g_down(F.linear(hidden_batch, weight[-D:]))
        if not commit and _all_decode(lengths):
            out = _decode_readout(self, q, output_gate, read_states, None)
            return out.view(T, self.value_dim), None
        if not commit:
            # host boundaries: the plan is built without a device-to-host copy
            samples = [0, *accumulate(int(n) for n in lengths)]
            q_hat = l2norm(q.reshape(1, T, H, D))
            mask = torch.zeros(len(lengths), dtype=torch.bool)
            plan = build_chunk_plan(samples, samples, WY_TILE_TOKENS, event_slice=samples, commit_mask=mask)
            read = memt_gdn2_read_fwd(q_hat, read_states, plan, self.read_scale, out_dtype=v.dtype)
            output = self.o_norm(read.reshape(-1, D), output_gate.reshape(-1, D))
            return output.view(T, self.value_dim), None
        erase, write, decay_latent = torch.split(
            F.linear(hidden_batch, weight[self._write_gate_slice]), self.write_gate_rows, dim=-1)
        decay = self.f_down(decay_latent)
        if self.fused_prologue:
            read, next_state = token_memory_packed_fused(
                q, k, v, decay, self.decay_bias, self.decay_scale_log, erase, write, read_states, write_states,
                lengths=lengths, scale=self.read_scale, chunk_tokens=self.chunk_tokens, num_heads=H)
        else:
            q_hat, k_til, beta, g = memory_prologue(q, k, decay, self.decay_bias, self.decay_scale_log, erase, write,
                                                    H)
            read, next_state = token_memory_packed(
                q_hat, k_til, v.reshape(1, T, H, D), g, beta, read_states, write_states, erase=None,
                lengths=lengths, scale=self.read_scale, chunk_tokens=self.chunk_tokens)
        output = self.o_norm(read.reshape(-1, D), output_gate.reshape(-1, D))
        return output.view(T, self.value_dim), next_state

    @torch.no_grad()
    def packed_slots(self, hidden_states, pool, read_slot, write_slot, *, lengths, commit):
        """``packed`` on a state pool in place: sample ``n`` reads
        ``pool[read_slot[n]]`` and, when committing, scans from
        ``pool[write_slot[n]]`` and leaves its final state there.  ``pool`` is
        ``[slots, H, D, D]`` or ``[slots, 1, H, D, D]`` fp32.  Returns the
        residual ``[T, H*D]`` bf16."""
        T, H, D = len(hidden_states), self.num_heads, self.head_dim
        if hidden_states.ndim != 2 or hidden_states.shape[1] != self.hidden_size or \
                hidden_states.dtype != torch.bfloat16 or not hidden_states.is_cuda:
            raise ValueError("Memory expects CUDA BF16 hidden states [tokens, hidden_size]")
        if not lengths or any(n <= 0 for n in lengths) or sum(lengths) != T:
            raise ValueError("Packed sample lengths must cover the hidden token rows")
        if pool.device != hidden_states.device or pool.dtype != torch.float32 or pool.shape[-3:] != (H, D, D):
            raise ValueError(f"Memory expects an FP32 state pool [slots, ..., {H}, {D}, {D}] on the hidden device")
        hidden_batch = hidden_states.unsqueeze(0)
        weight = self.in_proj.weight
        q, k, v = F.linear(hidden_batch, weight[: self.qkv_width]).split(self.qkv_rows, dim=-1)
        output_gate = self.g_down(F.linear(hidden_batch, weight[-D:]))
        if not commit and _all_decode(lengths):
            out = _decode_readout(self, q, output_gate, pool.view(-1, H, D, D), read_slot)
            return out.view(T, self.value_dim)
        if not commit:
            q_hat = l2norm(q.reshape(1, T, H, D))
            read = read_slots(q_hat, pool, read_slot, lengths, self.read_scale)
            output = self.o_norm(read.reshape(-1, D), output_gate.reshape(-1, D))
            return output.view(T, self.value_dim)
        erase, write, decay_latent = torch.split(
            F.linear(hidden_batch, weight[self._write_gate_slice]), self.write_gate_rows, dim=-1)
        decay = self.f_down(decay_latent)
        if self.fused_prologue:
            read = token_memory_packed_fused_slots(
                q, k, v, decay, self.decay_bias, self.decay_scale_log, erase, write, pool, read_slot, write_slot,
                lengths=lengths, scale=self.read_scale, chunk_tokens=self.chunk_tokens, num_heads=H)
        else:
            q_hat, k_til, beta, g = memory_prologue(q, k, decay, self.decay_bias, self.decay_scale_log, erase, write,
                                                    H)
            read = token_memory_packed_slots(q_hat, k_til, v.reshape(1, T, H, D), g, beta, pool, read_slot,
                                             write_slot, erase=None, lengths=lengths, scale=self.read_scale,
                                             chunk_tokens=self.chunk_tokens)
        output = self.o_norm(read.reshape(-1, D), output_gate.reshape(-1, D))
        return output.view(T, self.value_dim)

    def forward(self, hidden_states, initial_state, *, commit):
        """Single-request entry (models/qwen/layer.py:154-161)."""
        return self.packed(hidden_states, initial_state, lengths=[len(hidden_states)], commit=commit,
                           write_states=initial_state)


def _all_decode(lengths) -> bool:
    """A query batch of one token per sample (the decode step)."""
    return all(int(n) == 1 for n in lengths)


def _decode_readout(block, q, output_gate, states, slots):
    """Decode query path of either block in one kernel: ``l2norm(q)``, the
    snapshot read ``bf16(scale * q_hat . bf16(S))`` of each sample's state and
    ``o_norm`` with the output gate (the reference's l2norm -> reader ->
    o_norm chain for length-1 samples, same roundings).  ``q`` and
    ``output_gate`` are the projection rows ``[1, T, H*D]``; ``states``
    ``[N, H, D, D]`` read at row ``n`` (or pool ``[slots, H, D, D]`` read at
    ``slots[n]``)."""
    norm = block.o_norm
    return readout_decode(states, q, output_gate, norm.weight.to(torch.bfloat16), num_heads=block.num_heads,
                          scale=block.read_scale, eps=norm.variance_epsilon, softcap=norm.output_gate_softcap_limit,
                          gate_kind=norm.gate_kind, q_eps=1e-6, slot_idx=slots, state_bf16=True)


def _latent_norm(inputs, weight, eps):
    """RMS norm of a latent in fp32, back to the input dtype
    (models/deepseek/ops/compiled_tensor_ops.py:12-20)."""
    value = inputs.float() if inputs.dtype in (torch.bfloat16, torch.float16) else inputs
    return (value * torch.rsqrt(value.square().mean(-1, keepdim=True) + eps) * weight.to(value.dtype)).to(inputs.dtype)


class _LatentNorm(nn.Module):
    def __init__(self, rank, eps):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(rank))
        self.eps = eps


class DeepSeekMemoryBlock(nn.Module):
    """The Flash memory block, with the reference's parameter names and shapes
    (models/deepseek/layer.py:54-107).  ``memory_config`` needs
    ``hidden_size``, ``num_heads``, ``head_dim``, ``kv_groups``, ``q_rank``,
    ``kv_rank``, ``gate_rank``, ``chunk_tokens``, ``norm_eps`` and
    ``output_softcap``.  Every token reads the incoming state; a commit also
    returns the final state."""

    def __init__(self, memory_config, *, device=None, fused_prologue: bool = True):
        super().__init__()
        self.fused_prologue = fused_prologue
        c = memory_config
        self.hidden_size = c.hidden_size
        self.num_heads = c.num_heads
        self.head_dim = c.head_dim
        self.value_dim = c.num_heads * c.head_dim
        self.read_scale = c.head_dim ** -0.5
        self.kv_groups = c.kv_groups
        self.chunk_tokens = c.chunk_tokens
        self.norm_eps = c.norm_eps
        self.gate_rows = (c.gate_rank,) * 4
        self.qkv_rows = (c.q_rank, c.kv_groups * c.kv_rank, c.kv_groups * c.kv_rank)
        self.in_proj = nn.Linear(c.hidden_size, sum(self.qkv_rows) + sum(self.gate_rows), bias=False)
        self.q_norm = _LatentNorm(c.q_rank, c.norm_eps)
        self.q_up = nn.Linear(c.q_rank, self.value_dim, bias=False)
        group_width = self.value_dim // c.kv_groups
        self.k_group_up = nn.Parameter(torch.empty(c.kv_groups, group_width, c.kv_rank))
        self.v_group_up = nn.Parameter(torch.empty(c.kv_groups, group_width, c.kv_rank))
        self.k_group_norm = nn.Parameter(torch.ones(c.kv_groups, c.kv_rank))
        self.v_group_norm = nn.Parameter(torch.ones(c.kv_groups, c.kv_rank))
        self.b_up = nn.Linear(c.gate_rank, self.value_dim, bias=False)
        self.w_up = nn.Linear(c.gate_rank, self.value_dim, bias=False)
        self.f_down = nn.Linear(c.gate_rank, self.value_dim, bias=False)
        self.g_down = nn.Linear(c.gate_rank, self.value_dim, bias=True)
        self.decay_scale_log = nn.Parameter(torch.zeros(c.num_heads))
        self.decay_bias = nn.Parameter(torch.zeros(self.value_dim))
        self.o_norm = MemTRMSNormGated(c.head_dim, eps=c.norm_eps, output_gate_softcap_limit=c.output_softcap)
        self.to(device=device, dtype=torch.bfloat16)
        self.eval()

    def _group_expand(self, latent, weight, gain):
        """Per-group latent norm, then each group's up-projection
        (models/deepseek/ops/compiled_tensor_ops.py:28-39)."""
        groups, width, rank = weight.shape
        inputs = _latent_norm(latent.reshape(-1, groups, rank), gain, self.norm_eps)
        # bf16 bmm with both operands contiguous
        out = torch.bmm(inputs.transpose(0, 1).contiguous(), weight.transpose(1, 2).contiguous())
        return out.transpose(0, 1).reshape(*latent.shape[:-1], groups * width)

    def _project(self, hidden_states):
        """``(q, k, v, output_gate, erase, write, decay)`` raw projection rows
        [1, T, H*D] bf16 (models/deepseek/layer.py:109-151; the gates are formed
        by the prologue kernel)."""
        parts = self.in_proj(hidden_states.unsqueeze(0)).split((*self.qkv_rows, *self.gate_rows), dim=-1)
        q = F.linear(_latent_norm(parts[0], self.q_norm.weight, self.q_norm.eps), self.q_up.weight)
        k = self._group_expand(parts[1], self.k_group_up, self.k_group_norm)
        v = self._group_expand(parts[2], self.v_group_up, self.v_group_norm)
        erase = F.linear(parts[3], self.b_up.weight)
        write = F.linear(parts[4], self.w_up.weight)
        decay = F.linear(parts[5], self.f_down.weight)
        output_gate = F.linear(parts[6], self.g_down.weight, self.g_down.bias)
        return q, k, v, output_gate, erase, write, decay

    def _output(self, read, output_gate):
        T = read.shape[1]
        return self.o_norm(read.reshape(-1, self.head_dim), output_gate.reshape(-1, self.head_dim)).view(
            T, self.value_dim)

    @torch.no_grad()
    def packed(self, hidden_states, read_states, *, lengths, commit, write_states):
        """``(residual [T, H*D] bf16, next_state [N,H,D,D] fp32 | None)``
        (models/deepseek/layer.py:153-183)."""
        validate_packed_inputs(self, hidden_states, read_states, write_states, lengths)
        T, H, D = len(hidden_states), self.num_heads, self.head_dim
        q, k, v, output_gate, erase, write, decay = self._project(hidden_states)
        if not commit and _all_decode(lengths):
            return _decode_readout(self, q, output_gate, read_states, None).view(T, self.value_dim), None
        if not commit:
            q_hat = l2norm(q.reshape(1, T, H, D))
            read = snapshot_read(q_hat, read_states, lengths, self.read_scale, bf16_accumulator_output=True)
            return self._output(read, output_gate), None
        if self.fused_prologue:
            read, next_state = token_memory_packed_fused(
                q, k, v, decay, self.decay_bias, self.decay_scale_log, erase, write, read_states, write_states,
                lengths=lengths, scale=self.read_scale, chunk_tokens=self.chunk_tokens, num_heads=H)
            return self._output(read, output_gate), next_state
        q_hat, k_til, beta, g = memory_prologue(q, k, decay, self.decay_bias, self.decay_scale_log, erase, write, H,
                                                eps=1e-6)
        read, next_state = token_memory_packed_flash(
            q_hat, k_til, v.reshape(1, T, H, D), g, beta, read_states, write_states, lengths=lengths,
            scale=self.read_scale, chunk_tokens=self.chunk_tokens)
        return self._output(read, output_gate), next_state

    @torch.no_grad()
    def packed_slots(self, hidden_states, pool, read_slot, write_slot, *, lengths, commit):
        """``packed`` on a state pool in place (see ``QwenMemoryBlock.packed_slots``)."""
        T, H, D = len(hidden_states), self.num_heads, self.head_dim
        if hidden_states.ndim != 2 or hidden_states.shape[1] != self.hidden_size or \
                hidden_states.dtype != torch.bfloat16 or not hidden_states.is_cuda:
            raise ValueError("Memory expects CUDA BF16 hidden states [tokens, hidden_size]")
        if not lengths or any(n <= 0 for n in lengths) or sum(lengths) != T:
            raise ValueError("Packed sample lengths must cover the hidden token rows")
        if pool.device != hidden_states.device or pool.dtype != torch.float32 or pool.shape[-3:] != (H, D, D):
            raise ValueError(f"Memory expects an FP32 state pool [slots, ..., {H}, {D}, {D}] on the hidden device")
        q, k, v, output_gate, erase, write, decay = self._project(hidden_states)
        if not commit and _all_decode(lengths):
            return _decode_readout(self, q, output_gate, pool.view(-1, H, D, D), read_slot).view(T, self.value_dim)
        if not commit:
            read = read_slots(l2norm(q.reshape(1, T, H, D)), pool, read_slot, lengths, self.read_scale)
            return self._output(read, output_gate)
        if self.fused_prologue:
            read = token_memory_packed_fused_slots(
                q, k, v, decay, self.decay_bias, self.decay_scale_log, erase, write, pool, read_slot, write_slot,
                lengths=lengths, scale=self.read_scale, chunk_tokens=self.chunk_tokens, num_heads=H)
            return self._output(read, output_gate)
        q_hat, k_til, beta, g = memory_prologue(q, k, decay, self.decay_bias, self.decay_scale_log, erase, write, H,
                                                eps=1e-6)
        read = token_memory_packed_slots(q_hat, k_til, v.reshape(1, T, H, D), g, beta, pool, read_slot, write_slot,
                                         erase=None, lengths=lengths, scale=self.read_scale,
                                         chunk_tokens=self.chunk_tokens)
        return self._output(read, output_gate)

    def forward(self, hidden_states, initial_state, *, commit):
        """Single-request entry (models/deepseek/layer.py:190-198)."""
        return self.packed(hidden_states, initial_state, lengths=[len(hidden_states)], commit=commit,
                           write_states=initial_state)
