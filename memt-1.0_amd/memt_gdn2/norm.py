"""``MemTRMSNormGated`` on the HIP epilogue kernel (models/qwen/layer.py:15-31)."""

from __future__ import annotations

import torch
from torch import nn

from .ops import rms_norm_gated


class MemTRMSNormGated(nn.Module):
    """RMSNorm over the value dim, weight, then the SoftCapSiLU output gate
    ``c * tanh(silu(gate) / c)``; ``gate_kind="sigmoid"`` selects ``sigmoid(gate)``."""

    def __init__(self, hidden_size, *, eps, output_gate_softcap_limit, gate_kind: str = "softcap_silu"):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps
        self.output_gate_softcap_limit = float(output_gate_softcap_limit)
        self.gate_kind = gate_kind

    def forward(self, hidden_states, gate):
        return rms_norm_gated(hidden_states, gate, self.weight.to(torch.bfloat16), eps=self.variance_epsilon,
                              softcap=self.output_gate_softcap_limit, gate_kind=self.gate_kind)
