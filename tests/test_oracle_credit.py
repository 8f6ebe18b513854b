"""Pins of the credit-readout oracle (oracle/credit.py): the two-pass form against the dense definition, conservation,
the Q = 0 closed form and a brute-force double loop; a planted transpose must fail them."""
import pytest
import torch

from oracle import credit as oc


def _inputs(T=40, rows=2, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(rows, T, 64, generator=g, dtype=dtype)
    k = torch.randn(rows, T, 64, generator=g, dtype=dtype)
    e = torch.randn(rows, T, 64, generator=g, dtype=dtype)
    return q, k, e


@pytest.mark.parametrize('window', [0, 3, 17, 40])
def test_two_pass_equals_dense(window):
    q, k, e = _inputs()
    assert torch.allclose(oc.credit_two_pass(q, k, e, window), oc.credit_dense(q, k, e, window), atol=1e-10)


@pytest.mark.parametrize('window', [1, 9, 40])
def test_conservation(window):
    q, k, e = _inputs()
    c = oc.credit_dense(q, k, e, window)
    assert torch.allclose(c.sum(-2), e.sum(-2), atol=1e-9)


def test_q0_closed_form():
    q, k, e = _inputs()
    q = torch.zeros_like(q)
    for window in (0, 5, 39):
        assert torch.allclose(oc.credit_dense(q, k, e, window), oc.credit_q0_closed_form(e, window), atol=1e-10)


def test_bruteforce_double_loop():
    q, k, e = _inputs(T=12, rows=1)
    W = 4
    got = oc.credit_dense(q, k, e, W)[0]
    want = torch.zeros(12, 64, dtype=torch.float64)
    for s in range(12):
        ts = list(range(max(0, s - W), s + 1))
        logits = torch.stack([q[0, s] @ k[0, t] / 8 for t in ts])
        p = torch.softmax(logits, 0)
        for j, t in enumerate(ts):
            want[t] += p[j] * e[0, s]
    assert torch.allclose(got, want, atol=1e-12)


def test_lse_bruteforce():
    q, k, _ = _inputs(T=10, rows=1)
    got = oc.lse(q, k, 3)[0]
    for s in range(10):
        vals = torch.stack([q[0, s] @ k[0, t] / 8 for t in range(max(0, s - 3), s + 1)])
        assert abs(got[s].item() - torch.logsumexp(vals, 0).item()) < 1e-12


def test_planted_transpose_fails_conservation():
    """Using A instead of A^T breaks conservation (a plausible orientation mistake)."""
    q, k, e = _inputs()
    wrong = oc.attention_maps(q, k, 9) @ e
    assert not torch.allclose(wrong.sum(-2), e.sum(-2), atol=1e-6)


@pytest.mark.parametrize('window', [0, 5, 39])
def test_key_context_constant_values(window):
    """Every softmax row sums to 1, so constant values give center_s = hub_s . v exactly."""
    q, k, hub = _inputs()
    v = torch.randn(64, dtype=torch.float64)
    values = v.expand(2, 40, 64).clone()
    lse_, center = oc.key_context(q, k, values, hub, window)
    assert torch.allclose(center, hub @ v, atol=1e-10)
    assert torch.allclose(lse_, oc.lse(q, k, window), atol=1e-12)


def test_key_context_q0_closed_form():
    _, k, hub = _inputs()
    values = _inputs(seed=5)[2]
    q = torch.zeros(2, 40, 64, dtype=torch.float64)
    for window in (0, 7, 39):
        got = oc.key_context(q, k, values, hub, window)[1]
        assert torch.allclose(got, oc.key_context_q0_closed_form(values, hub, window), atol=1e-10)


def test_key_context_bruteforce():
    q, k, hub = _inputs(T=11, rows=1)
    values = _inputs(T=11, rows=1, seed=9)[0]
    W = 3
    lse_, center = oc.key_context(q, k, values, hub, W)
    for s in range(11):
        ts = range(max(0, s - W), s + 1)
        logits = torch.stack([q[0, s] @ k[0, t] / 8 for t in ts])
        p = torch.softmax(logits, 0)
        want = sum(p[j] * (hub[0, s] @ values[0, t]) for j, t in enumerate(ts))
        assert abs(center[0, s].item() - want.item()) < 1e-12
        assert abs(lse_[0, s].item() - torch.logsumexp(logits, 0).item()) < 1e-12


def test_planted_transposed_probabilities_fail():
    """center from p[t, s] instead of p[s, t] (a transposed softmax) breaks the constant-values identity."""
    q, k, hub = _inputs()
    v = torch.randn(64, dtype=torch.float64)
    values = v.expand(2, 40, 64).clone()
    lse_ = oc.lse(q, k, 9)
    logits = ((q @ k.transpose(-1, -2)) / 8).masked_fill(~oc._mask(40, 9), float('-inf'))
    p = torch.exp(logits - lse_.unsqueeze(-1))
    wrong = (p.transpose(-1, -2) * (hub @ values.transpose(-1, -2))).sum(-1)
    assert not torch.allclose(wrong, hub @ v, atol=1e-6)
    assert torch.allclose(oc.key_context(q, k, values, hub, 9)[1], hub @ v, atol=1e-10)


def test_by_token_layout():
    """Row r of the stacked layout is head r % H of layer r // H (moment_kernels.py:67-74), by explicit indexing."""
    x = torch.arange(6 * 5 * 4, dtype=torch.float64).reshape(6, 5, 4)
    H = 3
    bt = oc.by_token(x, H)
    for r in range(6):
        assert torch.equal(bt[r // H, :, (r % H) * 4:(r % H + 1) * 4], x[r])
    assert torch.equal(oc.stacked(bt, H), x)
