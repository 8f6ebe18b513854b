"""Cross-token credit readout on the MI355X windowed flash kernel.

credit_t = sum_{s in [t, t+W]} softmax_t'(q_s . k_t' / 8)[t] * e_s, the transpose of the causal attention map applied
to per-token error signals (train/val/run.py:965-985 attention_maps, :1095-1101 value_credit), computed in two passes
as the reference's production kernels do (train/speedrun/moment_kernels.py:79-110 lse, :612-661 value pass;
train/speedrun/value_gluon.py:145-172): an LSE pass over each query's window, then
out_t = sum_s exp(k_t . q_s / 8 - lse_s) src_s with bf16 probabilities, the source's bf16 high part (and optionally
its low part) and fp32 accumulation.

The ops are also registered as torch.library custom ops (noise_amd::credit_lse, noise_amd::raw_value_credits) with
fake kernels, the operator API the reference's kernels use (moment_kernels.py:664-673).
"""
from __future__ import annotations

import torch

from . import _lib


def _rows(t):
    if t.dim() != 3 or t.shape[-1] != 64:
        raise ValueError(f'expected (rows, T, 64), got {tuple(t.shape)}')
    return t.shape[0], t.shape[1]


def credit_lse(q: torch.Tensor, k: torch.Tensor, window: int) -> torch.Tensor:
    """lse [rows, T] of each query's window logits q_s . k_t / 8 (q, k: (rows, T, 64), cast to bf16)."""
    _lib.require_device(q, k)
    rows, T = _rows(q)
    q = q.to(torch.bfloat16).contiguous()
    k = k.to(torch.bfloat16).contiguous()
    lse = torch.empty(rows, T, dtype=torch.float32, device=q.device)
    _lib.call('noise_credit_lse', _lib.ptr(q), _lib.ptr(k), rows, T, int(window), _lib.ptr(lse), _lib.stream(q.device))
    return lse


def raw_value_credits(q: torch.Tensor, k: torch.Tensor, lse: torch.Tensor, hub: torch.Tensor, window: int,
                      hi_lo: bool = False) -> torch.Tensor:
    """sum_s p(s, t) hub_s for (rows, T, 64) inputs (moment_kernels.raw_value_credits): fp32 (rows, T, 64)."""
    _lib.require_device(q, k, lse, hub)
    rows, T = _rows(q)
    q = q.to(torch.bfloat16).contiguous()
    k = k.to(torch.bfloat16).contiguous()
    lse = lse.float().contiguous()
    hub = hub.float().contiguous()
    out = torch.empty(rows, T, 64, dtype=torch.float32, device=q.device)
    _lib.call('noise_credit_value', _lib.ptr(q), _lib.ptr(k), _lib.ptr(lse), _lib.ptr(hub), rows, T, int(window),
              int(bool(hi_lo)), _lib.ptr(out), _lib.stream(q.device))
    return out


def value_credit(q: torch.Tensor, k: torch.Tensor, hub: torch.Tensor, window: int, hi_lo: bool = False) -> torch.Tensor:
    """Both passes: A^T @ hub for A = softmax(mask(q k^T / 8)) (Boost.value_credit), (rows, T, 64) in and out."""
    return raw_value_credits(q, k, credit_lse(q, k, window), hub, window, hi_lo)


@torch.library.custom_op('noise_amd::credit_lse', mutates_args=())
def credit_lse_op(q: torch.Tensor, k: torch.Tensor, window: int) -> torch.Tensor:
    return credit_lse(q, k, window)


@credit_lse_op.register_fake
def _(q, k, window):
    return q.new_empty(q.shape[:2], dtype=torch.float32)


@torch.library.custom_op('noise_amd::raw_value_credits', mutates_args=())
def raw_value_credits_op(q: torch.Tensor, k: torch.Tensor, lse: torch.Tensor, hub: torch.Tensor,
                         window: int) -> torch.Tensor:
    return raw_value_credits(q, k, lse, hub, window)


@raw_value_credits_op.register_fake
def _(q, k, lse, hub, window):
    return torch.empty_like(hub, dtype=torch.float32)
