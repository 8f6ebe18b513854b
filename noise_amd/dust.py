"""Dust's head-slab CE estimator (train/val/dust.py:261-303, DUST.head_error) on the HIP kernels.

DUST.head_error(draws, sigma) reads three things from its DUST instance: the captured lm_head outputs of the clean
forward (self.outputs['lm_head']), the targets (self.y) and the clean per-token losses (self.clean_loss); it draws
its jitter from torch.randn (dust.py:192-193) and batches self.recipe.nrep draws per chunk. `head_error` here takes
those explicitly; the jitter is this library's counter stream, keyed by `seed` (the reference's CUDA generator
stream cannot be reproduced off an NVIDIA GPU), in fp32 where the reference rounds it and the reward-weighted sum
to bf16 (dust.py:281, 299-301).

    error = head_error(raw, y, clean_loss, draws=512, sigma=0.1)   # fp32, raw's shape; 0 past the vocabulary
"""
from __future__ import annotations

import torch

from . import _lib

SLAB = 256


def chunk_size(draws: int, cap: int) -> int:
    """The largest count up to cap that divides draws: that many draws share one chunk (dust.py:81-83)."""
    return next(n for n in range(min(cap, draws), 0, -1) if draws % n == 0)


def head_error(raw: torch.Tensor, y: torch.Tensor, clean_loss: torch.Tensor, draws: int, sigma: float = 0.1,
               nrep: int = 16, seed: int = 0, vocab: int | None = None) -> torch.Tensor:
    """Per-token error estimates of the lm_head outputs: raw (b, t, Vp) (cast to bf16, the autocast output the
    reference caches), y int (b, t) with -1 at ignored positions, clean_loss (b, t) the clean forward's per-token CE.
    Each chunk of chunk_size(draws, nrep) draws jitters one 256-column slab of the first `vocab` columns (default: all
    of Vp), in turn; the chunks must cover the slabs evenly, as the reference requires (dust.py:163)."""
    _lib.require_device(raw, y, clean_loss)
    if raw.dim() != 3 or y.shape != raw.shape[:2] or clean_loss.shape != raw.shape[:2]:
        raise ValueError('raw must be (b, t, Vp) with y and clean_loss (b, t)')
    b, t, Vp = raw.shape
    vocab = Vp if vocab is None else int(vocab)
    raw = raw.to(torch.bfloat16).contiguous()
    y = y.to(torch.int64).contiguous()
    clean_loss = clean_loss.float().contiguous()
    error = torch.empty(b, t, Vp, dtype=torch.float32, device=raw.device)
    ws = torch.empty(_lib.lib().noise_head_error_workspace(b * t, vocab, int(draws)), dtype=torch.uint8,
                     device=raw.device)
    _lib.call('noise_head_error', _lib.ptr(raw), Vp, _lib.ptr(y), _lib.ptr(clean_loss), b, t, vocab, int(draws),
              int(nrep), float(sigma), int(seed), _lib.ptr(error), _lib.ptr(ws), ws.numel(), _lib.stream(raw.device))
    return error
