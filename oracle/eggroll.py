"""ORACLE — test infrastructure only. CPU restatement of EGGROLL's per-step bookkeeping and update
(archive/10M/train/val/eggroll.py), fp32 numpy/torch on CPU:

  eggroll.py:117-128   offsets and noise slices     (counter-based generator: oracle/rng.c)
  eggroll.py:133-146   member layout                 direction (g // 2) % pairs, sign +sigma for even g, sequence of
                                                     the member's chunk start // per_seq
  eggroll.py:151-154   fitness                       f_j = L[2j+1] - L[2j]; f / (unbiased std + 1e-8);
                                                     weight[j % pairs] += f_j
  eggroll.py:155-166   gradient assembly             G = -(sum_j w_j a_j b_j^T) / len(f); 1-D: -(w @ eps) / len(f)
  eggroll.py:205       optimizer                     torch.optim.AdamW(lr, betas, eps=1e-8, weight_decay=0)

Parity pins (tests/test_oracle_eggroll.py): the layout against the reference's own arange/repeat_interleave algebra
run on small integers, the fitness against the textbook z-score, the gradient against a brute-force sum of outer
products, and adamw() against torch.optim.AdamW.
"""
from __future__ import annotations

import numpy as np
import torch

from . import rng
from .model import Config, param_specs

CHUNK = 256  # pairs per batched forward (eggroll.py:34)


def member_layout(pairs, n_seq, world=1, rank=0, chunk=CHUNK):
    """(direction, sign +1/-1, sequence) of every member this rank evaluates, in evaluation order."""
    members = max(2 * pairs, 2 * n_seq)
    per_seq, per_rank = members // n_seq, members // world
    direction, sign, seq = [], [], []
    for start in range(rank * per_rank, (rank + 1) * per_rank, 2 * chunk):
        for g in range(start, min(start + 2 * chunk, (rank + 1) * per_rank)):
            direction.append((g // 2) % pairs)
            sign.append(1 if g % 2 == 0 else -1)
            seq.append(start // per_seq)
    return np.array(direction), np.array(sign), np.array(seq)


def step_offsets(cfg: Config, seed, step, pairs):
    """name -> off [pairs] for every parameter (eggroll.py:117-120)."""
    return {name: rng.offsets(seed, step, p, int(sum(shape)), pairs)
            for p, (name, shape) in enumerate(param_specs(cfg))}


def noise(cfg: Config, seed, offsets, directions):
    """name -> (a [n, out], b [n, in]) or eps [n, L] as fp32 torch tensors (eggroll.py:122-128)."""
    out = {}
    for name, shape in param_specs(cfg):
        rows = torch.from_numpy(rng.rows(seed, offsets[name][directions], int(sum(shape))))
        out[name] = (rows[:, :shape[0]], rows[:, shape[0]:]) if len(shape) == 2 else rows
    return out


def fitness(losses):
    """z-scored antithetic differences (eggroll.py:151-152), torch.std's unbiased estimator."""
    losses = torch.as_tensor(losses, dtype=torch.float32)
    f = losses[1::2] - losses[0::2]
    return f / (f.std() + 1e-8)


def direction_weights(f, pairs):
    """weight[j % pairs] += f_j (eggroll.py:153-154)."""
    w = torch.zeros(pairs, dtype=torch.float32)
    return w.index_add_(0, torch.arange(len(f)) % pairs, f)


def gradients(cfg: Config, seed, offsets, weight, n_fitness):
    """name -> gradient (eggroll.py:155-166), summed in fp32 over every direction."""
    dirs = np.arange(len(weight))
    nz = noise(cfg, seed, offsets, dirs)
    out = {}
    for name, n in nz.items():
        if isinstance(n, tuple):
            g = -((weight[:, None] * n[0]).t() @ n[1])
        else:
            g = -(weight @ n)
        out[name] = g / n_fitness
    return out


def adamw(param, grad, m, v, step, lr, betas=(0.5, 0.95), eps=1e-8, weight_decay=0.0):
    """One AdamW update of fp32 tensors in place, torch.optim.AdamW's single-tensor arithmetic order."""
    b1, b2 = betas
    param.mul_(1 - lr * weight_decay)
    m.lerp_(grad, 1 - b1)
    v.mul_(b2).addcmul_(grad, grad, value=1 - b2)
    bc1 = 1 - b1 ** step
    bc2 = 1 - b2 ** step
    denom = (v.sqrt() / (bc2 ** 0.5)).add_(eps)
    param.addcdiv_(m, denom, value=-lr / bc1)
    return param
