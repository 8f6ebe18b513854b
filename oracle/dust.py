"""ORACLE — test infrastructure only. Nothing in the product path may import or call this module.

CPU restatement of Dust's head-slab CE estimator, DUST.head_error (train/val/dust.py:261-303), in fp32 torch, with
this build's counter-based jitter (oracle/rng.py head_noise) in place of the estimator's torch.randn draws
(dust.py:192-193, 281). Chunks of n = chunk_size(draws, nrep) draws (dust.py:81-83) each jitter one 256-column
slab of the cached lm_head outputs, in turn; a draw's loss is recomputed from the cached exponential sums of the
other slabs; rewards are the clean loss minus the draw's, zero at ignored targets, centered over the batch; the
error of the slab's columns accumulates -(reward / sigma) * jitter, and the result is divided by the draws per slab.

Pinned (tests/test_oracle_dust.py): the slab bookkeeping against a dense log-sum-exp of the jittered row, and, by
Stein's lemma, the estimate over many small-sigma draws against (1 - 1/b) times the analytic gradient of the
soft-capped CE with respect to the raw logits.
"""
from __future__ import annotations

import torch

from oracle import rng

SLAB = 256


def chunk_size(draws, cap):
    """The largest count up to cap that divides draws (dust.py:81-83)."""
    return next(n for n in range(min(cap, draws), 0, -1) if draws % n == 0)


def jitter(seed, draw, b, t):
    """float32 [b, t, 256]: draw `draw`'s jitter at token rows b * t + t' (row-major over batch and position)."""
    return torch.from_numpy(rng.head_noise(seed, draw, 0, b * t)).view(b, t, SLAB)


def head_error(raw, y, clean_loss, draws, sigma=0.1, nrep=16, seed=0, vocab=None):
    """raw float32 [b, t, Vp] (the lm_head outputs), y int64 [b, t] (-1: ignored), clean_loss float32 [b, t];
    returns the error estimate float32 [b, t, Vp] (zero past the vocabulary)."""
    b, t, Vp = raw.shape
    vocab = vocab or Vp
    n = chunk_size(draws, nrep)
    slabs = vocab // SLAB
    if (draws // n) % slabs:
        raise ValueError('the chunks of draws must cover the slabs evenly')
    logits = 15 * torch.tanh(raw[..., :vocab].float() / 15)
    slab_sums = logits.exp().view(b, t, slabs, SLAB).sum(-1)
    total = slab_sums.sum(-1)
    target = y.clamp(min=0)
    clean_target = logits.gather(-1, target.unsqueeze(-1)).squeeze(-1)
    target = target.repeat(n, 1)
    error = torch.zeros(b, t, Vp, dtype=torch.float32)
    for chunk in range(draws // n):
        block = chunk % slabs
        lo = block * SLAB
        a = torch.stack([jitter(seed, chunk * n + j, b, t) for j in range(n)])  # [n, b, t, 256]
        changed = raw[..., lo:lo + SLAB].float().repeat(n, 1, 1) + sigma * a.view(n * b, t, SLAB)
        changed = 15 * torch.tanh(changed / 15)
        partition = (total - slab_sums[..., block]).repeat(n, 1) + changed.exp().sum(-1)
        in_slab = (target >= lo) & (target < lo + SLAB)
        target_logit = torch.where(
            in_slab,
            changed.gather(-1, (target - lo).clamp(0, SLAB - 1).unsqueeze(-1)).squeeze(-1),
            clean_target.repeat(n, 1),
        )
        loss = (partition.log() - target_logit).view(n, b, t)
        reward = torch.where(y.unsqueeze(0) != -1, clean_loss.unsqueeze(0) - loss, torch.zeros(()))
        if b > 1:
            reward = reward - reward.mean(1, keepdim=True)
        error[..., lo:lo + SLAB] -= torch.einsum('nbt,nbtd->btd', reward / sigma, a)
    return error / (draws // slabs)


def soft_capped_ce(raw, y, vocab=None):
    """Per-token CE of the soft-capped logits (dust.py:94-99 after the head): float32 [b, t], 0 at ignored targets."""
    vocab = vocab or raw.shape[-1]
    z = 15 * torch.tanh(raw[..., :vocab].float() / 15)
    ce = torch.logsumexp(z, -1) - z.gather(-1, y.clamp(min=0).unsqueeze(-1)).squeeze(-1)
    return torch.where(y != -1, ce, torch.zeros(()))
