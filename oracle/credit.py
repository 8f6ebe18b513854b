"""ORACLE — test infrastructure only. CPU restatement of the cross-token credit readout.

  train/val/run.py:965-985     Boost.attention_maps  A = softmax_t(mask(q_s . k_t / 8)), mask 0 <= s - t <= W
  train/val/run.py:1095-1101   Boost.value_credit     credit = A^T @ hub (per batch and head)
  train/speedrun/moment_kernels.py:79-110    _implicit_key_statistics  lse_s over the window
  train/speedrun/moment_kernels.py:612-661   _value_credit_kernel      out_t = sum_{s in [t, t+W]} exp(k_t.q_s/8 - lse_s) src_s

All fp32 (float64 where asked) on CPU. Parity pins (tests/test_oracle_credit.py): the two-pass form against the dense
definition, conservation sum_t credit_t = sum_s hub_s, the Q = 0 closed form credit_t = sum_{s=t}^{min(t+W,T-1)}
hub_s / (min(s, W) + 1), and a brute-force double loop on tiny shapes.
"""
from __future__ import annotations

import torch


def _mask(T, window):
    pos = torch.arange(T)
    lag = pos[:, None] - pos[None, :]  # [query s, key t]
    return (lag >= 0) & (lag <= window)


def attention_maps(q, k, window):
    """q, k [..., T, D] (already normed / rotated) -> A [..., T(query), T(key)]."""
    T, D = q.shape[-2], q.shape[-1]
    logits = (q @ k.transpose(-1, -2)) / D ** 0.5
    return logits.masked_fill(~_mask(T, window), float('-inf')).softmax(-1)


def credit_dense(q, k, hub, window):
    """credit [..., T, C] = A^T @ hub."""
    return attention_maps(q, k, window).transpose(-1, -2) @ hub


def lse(q, k, window):
    """lse [..., T] over each query's window of keys, scale 1/8 for D = 64 (1/sqrt(D) in general)."""
    T, D = q.shape[-2], q.shape[-1]
    logits = (q @ k.transpose(-1, -2)) / D ** 0.5
    return torch.logsumexp(logits.masked_fill(~_mask(T, window), float('-inf')), -1)


def value_pass(q, k, lse_, src, window):
    """out_t = sum_s exp(k_t . q_s / sqrt(D) - lse_s) src_s over receivers s in [t, t + W]."""
    T, D = q.shape[-2], q.shape[-1]
    logits = (k @ q.transpose(-1, -2)) / D ** 0.5  # [key t, query s]
    p = torch.exp(logits - lse_.unsqueeze(-2)).masked_fill(~_mask(T, window).t(), 0.0)
    return p @ src


def credit_two_pass(q, k, src, window):
    return value_pass(q, k, lse(q, k, window), src, window)


def credit_q0_closed_form(hub, window):
    """credit when every logit is equal (Q = 0): A[s, t] = 1 / (min(s, W) + 1) on the window."""
    T = hub.shape[-2]
    scale = 1.0 / (torch.clamp(torch.arange(T), max=window) + 1.0).to(hub.dtype)
    weighted = hub * scale[:, None]
    out = torch.zeros_like(hub)
    for t in range(T):
        out[..., t, :] = weighted[..., t:min(t + window, T - 1) + 1, :].sum(-2)
    return out
