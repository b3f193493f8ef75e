"""The memory blocks keep the reference's parameter names and shapes, so a
checkpoint's state dict loads unchanged (models/qwen/layer.py:34-69,
models/deepseek/layer.py:54-107).  CPU only: construction touches no GPU."""

import types

import torch

from memt_gdn2.block import DeepSeekMemoryBlock, QwenMemoryBlock


def _shapes(block):
    return {name: tuple(p.shape) for name, p in block.state_dict().items()}


def test_qwen_block_state_dict():
    H, D, hidden = 16, 128, 1024
    cfg = types.SimpleNamespace(hidden_size=hidden, num_heads=H, head_dim=D, chunk_tokens=2048, rms_norm_eps=1e-6,
                                output_gate_softcap=2.0)
    block = QwenMemoryBlock(cfg)
    W = H * D
    assert _shapes(block) == {
        "in_proj.weight": (5 * W + 2 * D, hidden),  # q, k, v, erase, write, decay latent, output latent
        "f_down.weight": (W, D),
        "g_down.weight": (W, D),
        "decay_scale_log": (H,),
        "decay_bias": (W,),
        "o_norm.weight": (D,),
    }
    assert all(p.dtype == torch.bfloat16 for p in block.parameters())


def test_deepseek_block_state_dict():
    cfg = types.SimpleNamespace(hidden_size=4096, num_heads=64, head_dim=512, kv_groups=8, q_rank=1024, kv_rank=512,
                                gate_rank=256, chunk_tokens=2048, norm_eps=1e-6, output_softcap=2.0)
    block = DeepSeekMemoryBlock(cfg, device="meta")
    W = 64 * 512
    assert _shapes(block) == {
        "in_proj.weight": (1024 + 2 * 8 * 512 + 4 * 256, 4096),
        "q_norm.weight": (1024,),
        "q_up.weight": (W, 1024),
        "k_group_up": (8, W // 8, 512),
        "v_group_up": (8, W // 8, 512),
        "k_group_norm": (8, 512),
        "v_group_norm": (8, 512),
        "b_up.weight": (W, 256),
        "w_up.weight": (W, 256),
        "f_down.weight": (W, 256),
        "g_down.weight": (W, 256),
        "g_down.bias": (W,),
        "decay_scale_log": (64,),
        "decay_bias": (W,),
        "o_norm.weight": (512,),
    }
    assert block.read_scale == 512 ** -0.5 and block.gate_rows == (256,) * 4
    assert block.qkv_rows == (1024, 8 * 512, 8 * 512)
