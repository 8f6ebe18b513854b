"""AdamW on the fused HIP kernel: torch.optim.AdamW's update (archive/10M/train/val/eggroll.py:205, the foreach
arithmetic of torch 2.10) in one pass per parameter, optionally writing a bf16 copy of the updated weights."""
from __future__ import annotations

import torch

from . import _lib


class AdamW(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01):
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay))

    @torch.no_grad()
    def step(self, closure=None):
        loss = closure() if closure is not None else None
        for group in self.param_groups:
            b1, b2 = group['betas']
            for p in group['params']:
                if p.grad is None:
                    continue
                _lib.require_device(p)
                if p.dtype != torch.float32 or not p.is_contiguous():
                    raise ValueError('AdamW takes contiguous fp32 parameters')
                state = self.state[p]
                if not state:
                    state['step'] = 0
                    state['exp_avg'] = torch.zeros_like(p)
                    state['exp_avg_sq'] = torch.zeros_like(p)
                state['step'] += 1
                g = p.grad.float().contiguous()
                _lib.call('noise_adamw', _lib.ptr(p), _lib.ptr(g), _lib.ptr(state['exp_avg']),
                          _lib.ptr(state['exp_avg_sq']), p.numel(), group['lr'], b1, b2, group['eps'],
                          group['weight_decay'], state['step'], None, _lib.stream(p.device))
                p.add_(0.0)  # in-place no-op: bumps the version counter that cached bf16 weight copies key on
        return loss
