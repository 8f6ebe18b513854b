"""GPU parity of the head-slab CE estimator (noise_amd/dust.py, noise_head_error; train/val/dust.py:261-303) against
the fp32 oracle (oracle/dust.py) with the same counter-based jitter.

Tolerance: 1e-3 of the largest |error| (fp32 arithmetic on both sides; the sums run in different orders and tanh /
exp are different implementations). Columns past the vocabulary must be exactly 0."""
import pytest
import torch

from oracle import dust as od

pytestmark = pytest.mark.gpu


def _case(b, t, V, seed, vocab=None):
    vocab = vocab or V
    g = torch.Generator().manual_seed(seed)
    raw = (3.0 * torch.randn(b, t, V, generator=g)).to(torch.bfloat16).float()
    y = torch.randint(0, vocab, (b, t), generator=g)
    y.view(-1)[::7] = -1
    clean = od.soft_capped_ce(raw, y, vocab) + 0.01 * torch.randn(b, t, generator=g)  # the model's CE, slightly off
    return raw, y, clean


@pytest.mark.parametrize('b,t,vocab,Vp,draws,nrep', [
    (2, 64, 512, 512, 64, 16),   # 2 slabs, 4 chunks of 16
    (1, 128, 256, 320, 24, 16),  # 1 slab, chunks of 12, no centering, 64 padded columns
    (4, 32, 768, 768, 48, 8),    # 3 slabs, 6 chunks of 8
])
def test_head_error_matches_oracle(dev, b, t, vocab, Vp, draws, nrep):
    print(f'head_error b={b} t={t} vocab={vocab} ld={Vp} draws={draws} nrep={nrep}', flush=True)
    from noise_amd import dust
    raw, y, clean = _case(b, t, Vp, seed=b * 1000 + t, vocab=vocab)
    ref = od.head_error(raw, y, clean, draws, sigma=0.1, nrep=nrep, seed=9, vocab=vocab)
    got = dust.head_error(raw.to(dev), y.to(dev), clean.to(dev), draws, sigma=0.1, nrep=nrep, seed=9,
                          vocab=vocab).cpu()
    assert got.shape == ref.shape
    err = ((got - ref).abs().max() / ref.abs().max()).item()
    assert err < 1e-3, err
    assert torch.all(got[..., vocab:] == 0)


def test_head_error_rejects_uneven_slabs(dev):
    from noise_amd import dust
    raw, y, clean = _case(1, 16, 512, seed=1)
    with pytest.raises(ValueError):  # one chunk of 16 draws cannot cover 2 slabs
        dust.head_error(raw.to(dev), y.to(dev), clean.to(dev), 16, nrep=16)
