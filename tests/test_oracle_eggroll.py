"""Pins of the EGGROLL bookkeeping oracle (oracle/eggroll.py): member layout against the reference's own
arange / repeat_interleave algebra (eggroll.py:133-146, restated on integers), the textbook z-score, a brute-force sum
of outer products, and AdamW against torch.optim.AdamW."""
import math

import numpy as np
import pytest
import torch

from oracle import eggroll as oe
from oracle import model as om
from oracle import rng


def _reference_layout(pairs, n_seq, world, rank, chunk):
    """eggroll.py:133-146 with the same torch calls on integers (directions, sign pattern, sequence per chunk)."""
    members = max(2 * pairs, 2 * n_seq)
    per_seq, per_rank = members // n_seq, members // world
    dirs, signs, seqs = [], [], []
    sign = torch.tensor([1, -1]).repeat(chunk)
    for start in range(rank * per_rank, (rank + 1) * per_rank, 2 * chunk):
        directions = torch.arange(start, start + 2 * chunk, 2) % (2 * pairs) // 2
        dirs.append(directions.repeat_interleave(2, 0))
        signs.append(sign)
        seqs.append(torch.full((2 * chunk,), start // per_seq))
    return torch.cat(dirs).numpy(), torch.cat(signs).numpy(), torch.cat(seqs).numpy()


@pytest.mark.parametrize('pairs,n_seq,world,rank,chunk', [
    (12288, 8, 1, 0, 256), (12288, 8, 8, 3, 256), (128, 2, 1, 0, 64), (4, 8, 1, 0, 4), (96, 3, 2, 1, 16)])
def test_member_layout(pairs, n_seq, world, rank, chunk):
    d, s, q = oe.member_layout(pairs, n_seq, world, rank, chunk)
    rd, rs, rq = _reference_layout(pairs, n_seq, world, rank, chunk)
    assert np.array_equal(d, rd) and np.array_equal(s, rs) and np.array_equal(q, rq)


def test_fitness_textbook():
    r = np.random.default_rng(1)
    L = r.normal(8.3, 0.01, 64).astype(np.float32)
    f = oe.fitness(L).numpy()
    diff = L[1::2].astype(np.float64) - L[0::2]
    want = diff / (diff.std(ddof=1) + 1e-8)
    assert np.allclose(f, want, rtol=1e-4, atol=1e-5)
    w = oe.direction_weights(torch.from_numpy(f), 8).numpy()
    assert np.allclose(w, [f[j::8].sum() for j in range(8)], atol=1e-6)


def test_planted_biased_std_fails():
    r = np.random.default_rng(2)
    L = r.normal(0, 1, 16).astype(np.float32)
    diff = L[1::2].astype(np.float64) - L[0::2]
    wrong = diff / (diff.std(ddof=0) + 1e-8)
    assert not np.allclose(oe.fitness(L).numpy(), wrong, rtol=1e-4)


def test_gradient_bruteforce():
    cfg = om.Config(n_layer=2, sequence_len=128, vocab_size=128)
    pairs = 6
    offs = oe.step_offsets(cfg, 3, 1, pairs)
    weight = torch.linspace(-1.0, 1.0, pairs)
    grads = oe.gradients(cfg, 3, offs, weight, n_fitness=24)
    for name, shape in om.param_specs(cfg):
        width = int(sum(shape))
        rows = rng.rows(3, offs[name], width).astype(np.float64)
        want = np.zeros(shape)
        for j in range(pairs):
            if len(shape) == 2:
                want -= weight[j].item() * np.outer(rows[j, :shape[0]], rows[j, shape[0]:])
            else:
                want -= weight[j].item() * rows[j]
        assert np.allclose(grads[name].numpy(), want / 24, rtol=1e-4, atol=1e-6), name


@pytest.mark.parametrize('wd', [0.0, 0.1])
def test_adamw_matches_torch(wd):
    g = torch.Generator().manual_seed(4)
    p0 = torch.randn(1000, generator=g)
    ref_p = torch.nn.Parameter(p0.clone())
    opt = torch.optim.AdamW([ref_p], lr=1e-3, betas=(0.5, 0.95), eps=1e-8, weight_decay=wd, foreach=False)
    p, m, v = p0.clone(), torch.zeros(1000), torch.zeros(1000)
    for step in range(1, 6):
        grad = torch.randn(1000, generator=g)
        ref_p.grad = grad.clone()
        opt.step()
        oe.adamw(p, grad, m, v, step, lr=1e-3, weight_decay=wd)
    assert torch.equal(p, ref_p.data)
