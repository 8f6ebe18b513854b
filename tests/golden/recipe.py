"""Deterministic inputs shared by the golden-fixture writer (make_golden.py) and the tests that read the fixtures.

Weights and noise are drawn from the oracle's counter-based Gaussian buffer (oracle/rng.c, pinned by Philox
known-answer vectors), so a fixture only has to store outputs.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import rng
from oracle.eggroll import noise as oracle_noise, step_offsets
from oracle.model import Config, param_specs

SMALL = dict(sequence_len=64, vocab_size=256, n_layer=4, n_head=2, n_kv_head=2, n_embd=128, window_pattern='SSSL')
WEIGHT_SEED = 1234
TOKEN_SEED = 7


def weight_scale(name, shape):
    if name == 'resid_lambdas' or name == 'x0_lambdas':
        return 0.1
    if 'wte' in name or 'value_embeds' in name:
        return 1.0
    if 'lm_head' in name:
        return 0.05
    if 've_gate' in name:
        return 0.3
    return 1.0 / math.sqrt(shape[1])


def weights(cfg: Config, seed=WEIGHT_SEED):
    """name -> fp32 tensor: scale * G[base : base + numel] + (1 for resid_lambdas, 0.1 for x0_lambdas)."""
    out, base = {}, 0
    for name, shape in param_specs(cfg):
        n = math.prod(shape)
        w = rng.buffer(seed, base, n).reshape(shape) * weight_scale(name, shape)
        if name == 'resid_lambdas':
            w = w + 1.0
        elif name == 'x0_lambdas':
            w = w + 0.1
        out[name] = torch.from_numpy(np.ascontiguousarray(w, dtype=np.float32))
        base += n
    return out


def tokens(cfg: Config, batch, seed=TOKEN_SEED, ignore_every=0):
    """idx, targets int64 [batch, T] from a Zipf(1.1) inverse CDF over the vocabulary, driven by the buffer."""
    T = cfg.sequence_len
    u = (rng.buffer(seed, 0, batch * (T + 1)).astype(np.float64))
    u = 0.5 * (1.0 + np.vectorize(math.erf)(u / math.sqrt(2.0)))  # Gaussian -> uniform
    p = (np.arange(cfg.vocab_size) + 1.0) ** -1.1
    cdf = np.cumsum(p / p.sum())
    rows = np.minimum(np.searchsorted(cdf, u), cfg.vocab_size - 1).reshape(batch, T + 1)
    rows = torch.from_numpy(rows.astype(np.int64))
    idx, targets = rows[:, :-1].contiguous(), rows[:, 1:].contiguous()
    if ignore_every:
        targets.view(-1)[::ignore_every] = -1
    return idx, targets


def population_noise(cfg: Config, members, seed=WEIGHT_SEED + 1, step=3):
    """name -> per-member noise for `members` members (pairs share a direction) and the sign pattern."""
    pairs = members // 2
    offs = step_offsets(cfg, seed, step, pairs)
    dirs = np.arange(members) // 2
    return oracle_noise(cfg, seed, offs, dirs)
