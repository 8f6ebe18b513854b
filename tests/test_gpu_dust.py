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


# ---- the direct draws: capture, rerun and error sums (noise_dust_capture / _rerun / _errors; dust.py:195-259) ------

from oracle import model as om
from tests.golden import recipe

SEQ = 256
_ST = {}


def _setup(dev):
    if 'st' not in _ST:
        from tests.test_gpu_forward import _model
        from noise_amd.model import GPTConfig
        ocfg = om.Config(sequence_len=SEQ)
        w = recipe.weights(ocfg, seed=99)
        idx, tg = recipe.tokens(ocfg, batch=2, ignore_every=37)
        blocks, x0, clean = od.capture(w, ocfg, idx, tg)
        _ST['st'] = (ocfg, w, dict(blocks=blocks, x0=x0, idx=idx, targets=tg, clean=clean),
                     _model(dev, w, GPTConfig(sequence_len=SEQ)))
    return _ST['st']


def test_capture_matches_oracle(dev):
    print('dust capture B=2 T=256', flush=True)
    from noise_amd.dust import Dust
    ocfg, w, st, model = _setup(dev)
    d = Dust(model)
    clean = d.capture(st['idx'].to(dev), st['targets'].to(dev)).cpu()
    mask = st['targets'] >= 0
    assert ((clean - st['clean']).abs()[mask] / st['clean'][mask].abs()).max().item() < 1e-2
    assert torch.all(clean[~mask] == 0)
    for i in range(ocfg.n_layer):
        got, ref = d.blocks[i].cpu(), st['blocks'][i]
        assert ((got - ref).norm() / ref.norm()).item() < 1e-2, i
    assert ((d.x0.cpu() - st['x0']).norm() / st['x0'].norm()).item() < 1e-3


def test_capture_and_plain_forward_losses_are_bit_identical(dev):
    """The plain forward does not store block 0's input: block 0's attn c_proj rebuilds it from the recomputed x0 (the
    embedding kernel's operations). The capture stores it and reads it back. The per-token losses of the two paths
    must be the same bits."""
    print('dust capture vs plain forward B=2 T=256', flush=True)
    from noise_amd.dust import Dust
    from noise_amd.population import run_forward
    ocfg, w, st, model = _setup(dev)
    idx, tg = st['idx'].to(dev), st['targets'].to(dev)
    clean = Dust(model).capture(idx, tg)
    b, T = idx.shape
    seq = torch.arange(b, dtype=torch.int32, device=dev)
    out = run_forward(model, idx.contiguous(), tg.contiguous(), member_seq=seq, want_tokens=True, want_sum=False)
    torch.cuda.synchronize()
    assert torch.equal(out['token_loss'].view(b, T), clean)


@pytest.mark.parametrize('entry,sites', [
    (None, ['transformer.wte']),
    (0, ['o@0']),
    (1, ['transformer.h.1.attn.c_proj', 'transformer.h.1.mlp.c_proj']),  # the writers, jittered together
    (5, ['transformer.h.5.mlp.c_fc']),
    (7, ['transformer.h.7.mlp.c_proj']),
])
def test_rerun_matches_oracle(dev, entry, sites):
    print(f'dust rerun entry={entry} sites={sites}', flush=True)
    from noise_amd.dust import Dust
    ocfg, w, st, model = _setup(dev)
    d = Dust(model, seed=5)
    d.capture(st['idx'].to(dev), st['targets'].to(dev))
    got = d.rerun(3, entry, sites, 0.4, draw0=7).cpu()
    ref = od.rerun(w, ocfg, st, 3, entry, sites, 0.4, seed=d.seed, draw0=7)
    mask = (st['targets'] >= 0).expand(3, -1, -1)
    assert ((got - ref).abs()[mask] / ref[mask].abs()).max().item() < 1e-2
    assert (got - st['clean'].to(got)).abs().max() > 1e-3  # the jitter moved the losses


@pytest.mark.parametrize('gamma', [0.0, 0.3])
def test_error_sums_match_oracle_on_the_same_losses(dev, gamma):
    """The reward and error kernels against oracle/dust.py chunk_errors on the GPU's own per-token losses (1e-4 of the
    largest |error|: the same fp32 arithmetic in another order); then direct_errors equals its chunks' sum."""
    print(f'dust error sums gamma={gamma}', flush=True)
    from noise_amd import _lib
    from noise_amd.dust import Dust
    ocfg, w, st, model = _setup(dev)
    d = Dust(model, nrep=4, seed=2)
    d.capture(st['idx'].to(dev), st['targets'].to(dev))
    sites, entry, sigma = ['transformer.h.2.mlp.c_fc', 'transformer.h.2.attn.c_proj'], 2, 0.4
    chunks = []
    for d0 in (0, 4):
        loss = d.rerun(4, entry, sites, sigma, draw0=d0)
        chunks.append(loss.cpu())
        for name, key, width in [(sites[0], 'fc', 2048), (sites[1], 'attn', 512)]:
            err = torch.zeros(2, SEQ, width, device=dev)
            ws = torch.empty(_lib.lib().noise_dust_errors_workspace(4, 2, SEQ), dtype=torch.uint8, device=dev)
            _lib.call('noise_dust_errors', _lib.ptr(loss), _lib.ptr(d.clean_loss), 4, 2, SEQ, gamma, sigma, d.seed, d0,
                      od.SITE_ID[key], width, _lib.ptr(err), _lib.ptr(ws), ws.numel(), _lib.stream(dev))
            ref = od.chunk_errors(loss.cpu(), d.clean_loss.cpu(), sigma, gamma, d.seed, d0, key, width)
            assert (((err.cpu() - ref).abs().max()) / ref.abs().max()).item() < 1e-4, (name, d0)
    d.next_draw = 0
    est = d.direct_errors(sites, 8, sigma, entry=entry, gamma=gamma)
    for name, key, width in [(sites[0], 'fc', 2048), (sites[1], 'attn', 512)]:
        ref = sum(od.chunk_errors(c, d.clean_loss.cpu(), sigma, gamma, d.seed, d0, key, width)
                  for c, d0 in zip(chunks, (0, 4))) / 8
        assert (((est[name].cpu() - ref).abs().max()) / ref.abs().max()).item() < 1e-4, name
    assert d.next_draw == 8


def _oracle_inputs():
    if 'inputs' not in _ST:
        ocfg, w, st, _ = _ST['st']
        inputs = {}
        od.capture(w, ocfg, st['idx'], st['targets'], inputs=inputs)
        _ST['inputs'] = inputs
    return _ST['inputs']


def test_capture_keeps_the_writers_inputs(dev):
    """The capture's linear inputs (attention output, the MLP's normed input, relu² of c_fc; bf16 where the forward
    holds bf16) against the oracle's fp32 ones."""
    print('dust capture inputs B=2 T=256', flush=True)
    from noise_amd.dust import Dust
    ocfg, w, st, model = _setup(dev)
    d = Dust(model)
    d.capture(st['idx'].to(dev), st['targets'].to(dev))
    ref = _oracle_inputs()
    assert torch.equal(d.inputs['transformer.wte'].cpu(), st['idx'])
    for name, want in ref.items():
        if name == 'transformer.wte':
            continue
        got = d.inputs[name].float().cpu()
        assert ((got - want).norm() / want.norm()).item() < 1e-2, name


@pytest.mark.parametrize('site', ['transformer.h.1.attn.c_proj', 'transformer.h.1.mlp.c_fc',
                                  'transformer.h.6.mlp.c_proj', 'transformer.wte'])
def test_reassemble(dev, site):
    """reassemble against a float64 einsum / index_add on the GPU's own captured input (the kernel's arithmetic, 1e-4
    of the largest entry) and against the oracle's reassemble of its own input (1e-2 in norm)."""
    print(f'dust reassemble {site}', flush=True)
    from noise_amd.dust import Dust, parse_site
    ocfg, w, st, model = _setup(dev)
    d = Dust(model)
    d.capture(st['idx'].to(dev), st['targets'].to(dev))
    _, _, width = parse_site(model, site)
    err = torch.randn(2, SEQ, width, generator=torch.Generator().manual_seed(len(site)))
    got = d.reassemble(site, err.to(dev)).cpu().double()
    x = d.inputs[site].cpu()
    if site == 'transformer.wte':
        vocab = model.transformer.wte.weight.shape[0]
        exact = od.reassemble(x, err, vocab=vocab)
        oracle = od.reassemble(_oracle_inputs()[site], err, vocab=vocab)
    else:
        exact = od.reassemble(x.float(), err)
        oracle = od.reassemble(_oracle_inputs()[site], err)
    assert got.shape == exact.shape
    assert ((got - exact).abs().max() / exact.abs().max()).item() < 1e-4
    assert ((got - oracle).norm() / oracle.norm()).item() < 1e-2
