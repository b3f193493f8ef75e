"""Helpers shared by the GPU parity tests."""

import numpy as np
import torch


def to_dev(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to(dev, dtype) if dtype is not None else t.to(dev)


def bf(a, dev):
    return to_dev(np.asarray(a, np.float32), dev, torch.bfloat16)


def host(t):
    torch.cuda.synchronize()
    return t.detach().float().cpu().numpy()
