"""ORACLE — test infrastructure only. CPU restatement of the cross-token credit readout.

  train/val/run.py:965-985     Boost.attention_maps  A = softmax_t(mask(q_s . k_t / 8)), mask 0 <= s - t <= W
  train/val/run.py:1095-1101   Boost.value_credit     credit = A^T @ hub (per batch and head)
  train/speedrun/moment_kernels.py:79-110    _implicit_key_statistics  lse_s over the window
  train/speedrun/moment_kernels.py:612-661   _value_credit_kernel      out_t = sum_{s in [t, t+W]} exp(k_t.q_s/8 - lse_s) src_s
  train/speedrun/moment_kernels.py:79-110, 167-181  _implicit_key_statistics / _implicit_key_context
                                             center_s = sum_t p(s, t) (hub_s . v_t), p the window softmax of q_s . k_t / 8
  train/speedrun/moment_kernels.py:67-74     _by_token                 row r = head r % H of layer r // H (by-token layout)

All fp32 (float64 where asked) on CPU. Parity pins (tests/test_oracle_credit.py): the two-pass form against the dense
definition, conservation sum_t credit_t = sum_s hub_s, the Q = 0 closed form credit_t = sum_{s=t}^{min(t+W,T-1)}
hub_s / (min(s, W) + 1), and a brute-force double loop on tiny shapes. key_context: constant values give
center_s = hub_s . v exactly (softmax rows sum to 1), the Q = 0 closed form center_s = hub_s . mean_{t in window} v_t,
and a brute-force loop. by_token / stacked: a round trip and a brute-force index loop.
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


def key_context(q, k, values, hub, window):
    """(lse [..., T], center [..., T]): center_s = sum_t softmax_t(q_s . k_t / sqrt(D)) (hub_s . values_t)."""
    T, D = q.shape[-2], q.shape[-1]
    logits = ((q @ k.transpose(-1, -2)) / D ** 0.5).masked_fill(~_mask(T, window), float('-inf'))
    lse_ = torch.logsumexp(logits, -1)
    p = torch.exp(logits - lse_.unsqueeze(-1))
    scores = hub @ values.transpose(-1, -2)  # [receiver s, source t]
    return lse_, (p * scores).sum(-1)


def key_context_q0_closed_form(values, hub, window):
    """center when every logit is equal (Q = 0): hub_s . mean of values_t over t in [s - W, s]."""
    T = values.shape[-2]
    out = torch.empty(values.shape[:-1], dtype=values.dtype)
    for s in range(T):
        mean = values[..., max(0, s - window):s + 1, :].mean(-2)
        out[..., s] = (hub[..., s, :] * mean).sum(-1)
    return out


def by_token(stacked, heads):
    """(rows, T, C) -> (rows // heads, T, heads * C): row r is head r % heads of layer r // heads."""
    rows, T, C = stacked.shape
    return stacked.reshape(rows // heads, heads, T, C).transpose(1, 2).reshape(rows // heads, T, heads * C)


def stacked(by_tok, heads):
    """Inverse of by_token."""
    L, T, HC = by_tok.shape
    C = HC // heads
    return by_tok.reshape(L, T, heads, C).transpose(1, 2).reshape(L * heads, T, C)
