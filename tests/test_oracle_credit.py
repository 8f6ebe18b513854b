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
