"""Cross-token credit readout on the MI355X windowed flash kernel.

credit_t = sum_{s in [t, t+W]} softmax_t'(q_s . k_t' / 8)[t] * e_s, the transpose of the causal attention map applied
to per-token error signals (train/val/run.py:965-985 attention_maps, :1095-1101 value_credit), computed in two passes
as the reference's production kernels do (train/speedrun/moment_kernels.py:79-110 lse, :612-661 value pass;
train/speedrun/value_gluon.py:145-172): an LSE pass over each query's window, then
out_t = sum_s exp(k_t . q_s / 8 - lse_s) src_s with bf16 probabilities, the source's bf16 high part (and optionally
its low part) and fp32 accumulation.

The key-context pass (moment_kernels.py:79-110, 137-194) returns lse and center_s = sum_t p(s, t) (hub_s . v_t) in
one launch (key_context). value_pass takes exactly the arguments of moment_kernels._value_pass (:645-661), so it plugs
into the reference's VALUE_IMPL hook (:642-643, set at train/speedrun/run.py:1678) and serves every value-credit op
behind it, stacked and by-token layouts alike.

The ops are also registered as torch.library custom ops (noise_amd::credit_lse, noise_amd::raw_value_credits,
noise_amd::implicit_key_context_edges) with fake kernels, the operator API the reference's kernels use
(moment_kernels.py:184-194, 664-673).
"""
from __future__ import annotations

import torch

from . import _lib


def _rows(t):
    if t.dim() != 3 or t.shape[-1] != 64:
        raise ValueError(f'expected (rows, T, 64), got {tuple(t.shape)}')
    return t.shape[0], t.shape[1]


def _match(q, **others):
    """Every other operand on q's device with the shape its name implies: (rows, T, 64), or (rows, T) for lse."""
    rows, T = _rows(q)
    for name, t in others.items():
        want = (rows, T) if name == 'lse' else (rows, T, 64)
        if tuple(t.shape) != want:
            raise ValueError(f'{name} {tuple(t.shape)} does not match q {tuple(q.shape)}: expected {want}')
        if t.device != q.device:
            raise ValueError(f'{name} is on {t.device}, q on {q.device}')
        if not t.is_floating_point():
            raise ValueError(f'{name} must be floating point, got {t.dtype}')
    return rows, T


def credit_lse(q: torch.Tensor, k: torch.Tensor, window: int, bounded: bool = False) -> torch.Tensor:
    """lse [rows, T] of each query's window logits q_s . k_t / 8 (q, k: (rows, T, 64), cast to bf16). bounded: the
    caller guarantees |q_s . k_t| / 8 <= 16 on every in-window pair (RMS-normed q and k give <= 8); the pass then keeps
    no running maximum (noise_credit_lse_bounded): the sum of exp(logit) cannot overflow fp32 at any window, and the
    one extra bf16 rounding of q (it carries the scale) moves a logit by at most 16 * 2^-9 = 0.03."""
    rows, T = _match(q, k=k)
    _lib.require_device(q, k)
    q = q.to(torch.bfloat16).contiguous()
    k = k.to(torch.bfloat16).contiguous()
    lse = torch.empty(rows, T, dtype=torch.float32, device=q.device)
    _lib.call('noise_credit_lse_bounded' if bounded else 'noise_credit_lse', _lib.ptr(q), _lib.ptr(k), rows, T,
              int(window), _lib.ptr(lse), _lib.stream(q.device))
    return lse


def raw_value_credits(q: torch.Tensor, k: torch.Tensor, lse: torch.Tensor, hub: torch.Tensor, window: int,
                      hi_lo: bool = True) -> torch.Tensor:
    """sum_s p(s, t) hub_s for (rows, T, 64) inputs (moment_kernels.raw_value_credits): fp32 (rows, T, 64). The
    source enters as bf16 high and low parts, as the reference's Triton kernel always does (moment_kernels.py:633-636);
    hi_lo=False takes the high part only (value_gluon's HI mode)."""
    rows, T = _match(q, k=k, lse=lse, hub=hub)
    _lib.require_device(q, k, lse, hub)
    q = q.to(torch.bfloat16).contiguous()
    k = k.to(torch.bfloat16).contiguous()
    lse = lse.float().contiguous()
    hub = hub.float().contiguous()
    out = torch.empty(rows, T, 64, dtype=torch.float32, device=q.device)
    _lib.call('noise_credit_value', _lib.ptr(q), _lib.ptr(k), _lib.ptr(lse), _lib.ptr(hub), rows, T, int(window),
              int(bool(hi_lo)), _lib.ptr(out), _lib.stream(q.device))
    return out


def key_context(q: torch.Tensor, k: torch.Tensor, values: torch.Tensor, hub: torch.Tensor,
                window: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(lse, center) [rows, T] fp32 of each receiver's window (moment_kernels._implicit_key_context): lse as
    credit_lse, center_s = sum_t softmax_t(q_s . k_t / 8) (hub_s . values_t). Inputs (rows, T, 64), cast to bf16
    (the speedrun feeds bf16 copies, train/speedrun/run.py:1770-1771); fp32 probabilities and sums."""
    rows, T = _match(q, k=k, values=values, hub=hub)
    _lib.require_device(q, k, values, hub)
    q, k, values, hub = (t.to(torch.bfloat16).contiguous() for t in (q, k, values, hub))
    lse = torch.empty(rows, T, dtype=torch.float32, device=q.device)
    center = torch.empty_like(lse)
    _lib.call('noise_credit_key_context', _lib.ptr(q), _lib.ptr(k), _lib.ptr(values), _lib.ptr(hub), rows, T,
              int(window), _lib.ptr(lse), _lib.ptr(center), _lib.stream(q.device))
    return lse, center


# HI: the value source's bf16 high part only, as value_gluon's CONFIG['HI'] (train/speedrun/value_gluon.py:20-21);
# the default 0 adds the low part, as moment_kernels' Triton value kernel always does (moment_kernels.py:633-636).
CONFIG = dict(HI=0)


def value_pass(q, k, lse, source, window, in_heads=1, out_heads=1, out=None, layers=None, **over):
    """moment_kernels._value_pass's arguments and result (train/speedrun/moment_kernels.py:645-661).

    q, k (rows, T, 64); lse (rows, T); source stacked (rows, T, 64) or, with in_heads > 1, by token
    (rows // in_heads, T, >= in_heads * 64) with row r = head r % in_heads of layer r // in_heads; the output stacked
    or, with out_heads > 1, by token likewise, written into `out` (such a view, last stride 1) when given, layer l at
    index layers[l] of its first axis when `layers` (int32) is given. Returns the output. The kernel reads the source
    and writes the output in these layouts directly (noise_credit_value_strided)."""
    h, t, d = q.shape
    channels = source.shape[-1] // in_heads
    if d != 64 or channels != 64:
        raise ValueError(f'value_pass: head_dim {d} and source channels {channels} must be 64')
    if source.stride(-1) != 1 or (out is not None and out.stride(-1) != 1):
        raise AssertionError('value_pass: source and out need last stride 1')
    if h % in_heads or h % out_heads:
        raise ValueError(f'value_pass: {h} rows do not split into {in_heads} / {out_heads} heads')
    cfg = dict(CONFIG, **over)
    _match(q, k=k, lse=lse)
    _lib.require_device(q, k, lse, source)
    q = q.to(torch.bfloat16).contiguous()
    k = k.to(torch.bfloat16).contiguous()
    lse = lse.float().contiguous()
    src = source if source.dtype == torch.float32 else source.float()
    if src.stride(-1) != 1 or src.stride(0) % 4 or src.stride(1) % 4:
        src = src.contiguous()
    if src.shape[0] * in_heads != h or src.shape[1] != t:
        raise ValueError(f'value_pass: source {tuple(source.shape)} does not hold {h} rows of {t} tokens by {in_heads}')
    rows_map = None
    if out is None:
        out = torch.empty(h // out_heads, t, out_heads * 64, dtype=torch.float32, device=q.device)
    if out.dtype != torch.float32 or out.device != q.device or out.shape[1] != t or out.shape[-1] < out_heads * 64:
        raise ValueError(f'value_pass: out must be fp32 (n, {t}, >= {out_heads * 64}) on {q.device}')
    if layers is not None:
        rows_map = layers.to(device=q.device, dtype=torch.int32).contiguous()
        if rows_map.numel() != h // out_heads:
            raise ValueError(f'value_pass: {rows_map.numel()} layers for {h // out_heads} output rows')
        lo, hi = int(rows_map.min()), int(rows_map.max())
        if lo < 0 or hi >= out.shape[0]:
            raise IndexError(f'value_pass: layers index rows {lo}..{hi} of an output with {out.shape[0]}')
    elif out.shape[0] != h // out_heads:
        raise ValueError(f'value_pass: out has {out.shape[0]} rows, the pass writes {h // out_heads}')
    if out.stride(0) % 4 or out.stride(1) % 4:
        raise ValueError('value_pass: out strides must be multiples of 4 elements')
    _lib.call('noise_credit_value_strided', _lib.ptr(q), _lib.ptr(k), _lib.ptr(lse), _lib.ptr(src), in_heads,
              src.stride(0), src.stride(1), h, t, int(window), int(not cfg['HI']), _lib.ptr(out), out_heads,
              out.stride(0), out.stride(1), _lib.ptr(rows_map), _lib.stream(q.device))
    return out


def value_credit(q: torch.Tensor, k: torch.Tensor, hub: torch.Tensor, window: int, hi_lo: bool = True,
                 bounded: bool = False) -> torch.Tensor:
    """Both passes: A^T @ hub for A = softmax(mask(q k^T / 8)) (Boost.value_credit), (rows, T, 64) in and out.
    bounded: as credit_lse's."""
    return raw_value_credits(q, k, credit_lse(q, k, window, bounded), hub, window, hi_lo)


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


@torch.library.custom_op('noise_amd::implicit_key_context_edges', mutates_args=())
def implicit_key_context_edges_op(q: torch.Tensor, k: torch.Tensor, values: torch.Tensor, hub: torch.Tensor,
                                  window: int) -> tuple[torch.Tensor, torch.Tensor]:
    return key_context(q, k, values, hub, window)


@implicit_key_context_edges_op.register_fake
def _(q, k, values, hub, window):
    h, t, _ = q.shape
    return q.new_empty((h, t), dtype=torch.float32), q.new_empty((h, t), dtype=torch.float32)
