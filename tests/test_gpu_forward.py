"""GPU parity of the fixed GPT's forward and of the population forward against the fp32 oracle.

Tolerance: per-token / per-member losses within 1e-2 relative (bf16 operands, fp32 accumulation), the path's
stated bound for per-member losses."""
import numpy as np
import pytest
import torch

from oracle import model as om
from tests.golden import recipe

pytestmark = pytest.mark.gpu

SEQ = 256  # windows 128 (S) and 256 (L) at sequence_len 256


def _cfgs():
    ocfg = om.Config(sequence_len=SEQ)
    from noise_amd.model import GPTConfig
    return ocfg, GPTConfig(sequence_len=SEQ)


_W = {}


def _weights(ocfg):
    if SEQ not in _W:
        _W[SEQ] = recipe.weights(ocfg, seed=99)
    return _W[SEQ]


def _model(dev, w, gcfg):
    from noise_amd.model import GPT
    with torch.device('meta'):
        model = GPT(gcfg)
    model.to_empty(device=dev)
    model.init_weights()
    model.transformer.wte.float()
    for e in model.value_embeds.values():
        e.float()
    model.load_state_dict({k: v.to(dev) for k, v in w.items()}, strict=True)
    return model


def test_gpt_forward_matches_oracle(dev):
    print('gpt forward B=2 T=256', flush=True)
    ocfg, gcfg = _cfgs()
    w = _weights(ocfg)
    model = _model(dev, w, gcfg)
    idx, tg = recipe.tokens(ocfg, batch=2, ignore_every=37)
    ref = om.gpt_forward(w, ocfg, idx, tg, 'none')
    got = model(idx.to(dev), tg.to(dev), loss_reduction='none').cpu()
    mask = tg.reshape(-1) >= 0
    rel = ((got - ref).abs()[mask] / ref[mask].abs()).max().item()
    assert rel < 1e-2, rel
    assert torch.all(got[~mask] == 0)
    s = model(idx.to(dev), tg.to(dev), loss_reduction='sum').item()
    assert abs(s - ref.sum().item()) / ref.sum().item() < 1e-2
    mean = model(idx.to(dev), tg.to(dev)).item()
    assert abs(mean - ref.sum().item() / mask.sum().item()) / mean < 1e-2
    logits = model(idx.to(dev)).cpu()
    lref = om.gpt_forward(w, ocfg, idx)
    assert ((logits - lref).abs().max() / lref.abs().max()).item() < 2e-2


def test_gpt_forward_vocab_not_a_tile_multiple(dev):
    """Vocabulary 1000 (table padded to 1024): the head's last 256-column tile holds 232 vocabulary columns and takes
    the CE epilogue's column-checked path, the other tiles its unchecked one (targets fall in both); per-token losses
    within 1e-2 of the oracle's."""
    from noise_amd.model import GPTConfig
    print('gpt forward vocab 1000 B=2 T=256', flush=True)
    ocfg = om.Config(sequence_len=SEQ, vocab_size=1000)
    w = recipe.weights(ocfg, seed=98)
    model = _model(dev, w, GPTConfig(sequence_len=SEQ, vocab_size=1000))
    idx, tg = recipe.tokens(ocfg, batch=2, seed=33, ignore_every=41)
    assert (tg >= 768).any() and ((tg >= 0) & (tg < 768)).any()
    ref = om.gpt_forward(w, ocfg, idx, tg, 'none')
    got = model(idx.to(dev), tg.to(dev), loss_reduction='none').cpu()
    mask = tg.reshape(-1) >= 0
    rel = ((got - ref).abs()[mask] / ref[mask].abs()).max().item()
    assert rel < 1e-2, rel
    assert torch.all(got[~mask] == 0)


def test_gpt_forward_short_sequence_padding(dev):
    """T = 100 (not a multiple of 128) is padded on the right; causal attention keeps the real positions exact."""
    ocfg, gcfg = _cfgs()
    w = _weights(ocfg)
    model = _model(dev, w, gcfg)
    idx, tg = recipe.tokens(ocfg, batch=1)
    idx, tg = idx[:, :100], tg[:, :100]
    ref = om.gpt_forward(w, ocfg, idx, tg, 'none')
    got = model(idx.to(dev), tg.to(dev), loss_reduction='none').cpu()
    assert got.shape == ref.shape
    assert ((got - ref).abs() / ref.abs()).max().item() < 1e-2


def test_population_loss_matches_oracle(dev):
    from noise_amd.population import population_loss
    print('population loss m=16 T=256', flush=True)
    ocfg, gcfg = _cfgs()
    w = _weights(ocfg)
    model = _model(dev, w, gcfg)
    members, sigma = 16, 0.05
    noise = recipe.population_noise(ocfg, members, seed=77, step=2)
    sign = torch.tensor([sigma, -sigma] * (members // 2))
    idx, tg = recipe.tokens(ocfg, batch=1, seed=31)
    ref = om.population_loss(w, ocfg, noise, sign, idx[0], tg[0]) / SEQ
    dnoise = {k: tuple(t.to(dev) for t in v) if isinstance(v, tuple) else v.to(dev) for k, v in noise.items()}
    got = population_loss(model, None, dnoise, sign.to(dev), idx[0].to(dev), tg[0].to(dev)).cpu()
    rel = ((got - ref).abs() / ref.abs()).max().item()
    assert rel < 1e-2, (got, ref)
    # the antithetic differences (the fitness signal) follow the oracle's: correlation over the 8 pairs
    d_ref, d_got = (ref[1::2] - ref[0::2]).numpy(), (got[1::2] - got[0::2]).numpy()
    assert np.corrcoef(d_ref, d_got)[0, 1] > 0.9, (d_ref, d_got)


def test_population_embedding_noise_reaches_every_mix(dev):
    """Only the embedding perturbed (sigma 2), and every block's lambda mix weighting x0 by 1: the antithetic loss
    differences then carry x0's perturbation through every mix, which the kernels recompute from the embedding table
    in the MLP projection's epilogue. A recompute without the member's noise term (planted in the oracle: the mixes
    of blocks 1..7 with the unperturbed x0) moves these differences by up to 0.08; the bound is 0.01."""
    from noise_amd.population import population_loss
    print('population loss, embedding noise only, m=8 T=256', flush=True)
    ocfg, gcfg = _cfgs()
    w = dict(_weights(ocfg))
    w['x0_lambdas'] = torch.ones_like(w['x0_lambdas'])
    model = _model(dev, w, gcfg)
    members, sigma = 8, 2.0
    noise = recipe.population_noise(ocfg, members, seed=78, step=1)
    wte = 'transformer.wte.weight'
    noise = {k: v if k == wte else (tuple(torch.zeros_like(t) for t in v) if isinstance(v, tuple) else torch.zeros_like(v))
             for k, v in noise.items()}
    sign = torch.tensor([sigma, -sigma] * (members // 2))
    idx, tg = recipe.tokens(ocfg, batch=1, seed=32)
    ref = om.population_loss(w, ocfg, noise, sign, idx[0], tg[0]) / SEQ
    dnoise = {k: tuple(t.to(dev) for t in v) if isinstance(v, tuple) else v.to(dev) for k, v in noise.items()}
    got = population_loss(model, None, dnoise, sign.to(dev), idx[0].to(dev), tg[0].to(dev)).cpu()
    assert ((got - ref).abs() / ref.abs()).max().item() < 1e-2, (got, ref)
    d_ref, d_got = ref[0::2] - ref[1::2], got[0::2] - got[1::2]
    print('antithetic differences', d_ref.tolist(), d_got.tolist(), flush=True)
    assert (d_got - d_ref).abs().max().item() < 0.01, (d_got, d_ref)


def test_lowrank_matches_bruteforce(dev):
    """x (W + s a b^T)^T with the perturbed weight materialized, on the CPU."""
    from noise_amd.population import lowrank
    g = torch.Generator().manual_seed(5)
    m, T, n_in, n_out = 3, 128, 512, 256
    x = torch.randn(m, T, n_in, generator=g).bfloat16().float()
    W = (torch.randn(n_out, n_in, generator=g) * 0.05).bfloat16().float()
    a, b = torch.randn(m, n_out, generator=g), torch.randn(m, n_in, generator=g)
    sign = torch.tensor([0.01, -0.01, 0.02])
    ref = torch.stack([x[i] @ (W + sign[i] * torch.outer(a[i], b[i])).t() for i in range(m)])
    got = lowrank(x.to(dev), W.to(dev), a.to(dev), b.to(dev), sign.to(dev)).cpu()
    assert ((got - ref).abs().max() / ref.abs().max()).item() < 1e-2


def test_lowrank_embed_matches_oracle(dev):
    """The perturbed embedding (eggroll.py:61-63) against oracle/model.py lowrank_embed: fp32 table to 1e-6 relative
    (one fma per value), bf16 table exactly on its fp32 values; an id outside the table gives a NaN row."""
    from noise_amd.population import lowrank_embed
    g = torch.Generator().manual_seed(8)
    V, d, m, T = 300, 512, 5, 77
    W = torch.randn(V, d, generator=g)
    a, b = torch.randn(m, V, generator=g), torch.randn(m, d, generator=g)
    idx = torch.randint(0, V, (T,), generator=g)
    sign = torch.tensor([0.01, -0.01, 0.02, -0.02, 0.5])
    ref = om.lowrank_embed(W, a, b, idx, sign)
    got = lowrank_embed(W.to(dev), a.to(dev), b.to(dev), idx.to(dev), sign.to(dev)).cpu()
    assert got.shape == (m, T, d)
    assert ((got - ref).abs().max() / ref.abs().max()).item() < 1e-6
    Wb = W.bfloat16()
    got_b = lowrank_embed(Wb.to(dev), a.to(dev), b.to(dev), idx.to(dev), sign.to(dev)).cpu()
    ref_b = om.lowrank_embed(Wb.float(), a, b, idx, sign)
    assert ((got_b - ref_b).abs().max() / ref_b.abs().max()).item() < 1e-6
    bad = idx.clone()
    bad[3] = V
    got_bad = lowrank_embed(W.to(dev), a.to(dev), b.to(dev), bad.to(dev), sign.to(dev)).cpu()
    assert torch.isnan(got_bad[:, 3]).all() and torch.isfinite(got_bad[:, :3]).all()


def test_hooked_forward_runs_module_by_module(dev):
    """Hooks on every Linear and Embedding and pre-hooks on the blocks, as Dust's capture registers them
    (train/val/dust.py:149-168): GPT.forward then runs the submodules, every hook sees its module once per call with
    the reference's shapes, and the per-token losses match the oracle's (and the fused path's) within 1e-2; the
    lengths include one that is not a multiple of 128 (the attention pads it)."""
    from torch import nn
    print('hooked GPT.forward B=2 T=256 and T=200', flush=True)
    ocfg, gcfg = _cfgs()
    w = _weights(ocfg)
    model = _model(dev, w, gcfg)
    idx, tg = recipe.tokens(ocfg, batch=2, seed=51)
    fused = model(idx.to(dev), tg.to(dev), loss_reduction='none').cpu()
    seen, blocks = {}, {}
    mods = {n: m for n, m in model.named_modules() if isinstance(m, (nn.Linear, nn.Embedding))}
    hooks = [m.register_forward_hook(lambda m, a, o, n=n: seen.setdefault(n, []).append((a[0].shape, o.shape)))
             for n, m in mods.items()]
    hooks += [b.register_forward_pre_hook(lambda m, a, i=i: blocks.setdefault(i, []).append(a[0].shape))
              for i, b in enumerate(model.transformer.h)]
    try:
        for T in (SEQ, 200):
            seen.clear()
            blocks.clear()
            got = model(idx[:, :T].to(dev), tg[:, :T].to(dev), loss_reduction='none').cpu()
            ref = om.gpt_forward(w, ocfg, idx[:, :T], tg[:, :T], 'none')
            assert ((got - ref).abs() / ref.abs()).max().item() < 1e-2
            assert set(seen) == set(mods) and all(len(v) == 1 for v in seen.values())
            assert seen['lm_head'][0][1] == (2, T, model.lm_head.weight.shape[0])
            assert seen['transformer.h.0.mlp.c_fc'][0] == ((2, T, 512), (2, T, 2048))
            assert sorted(blocks) == list(range(ocfg.n_layer)) and all(v == [(2, T, 512)] for v in blocks.values())
            if T == SEQ:
                assert ((got - fused).abs() / fused.abs()).max().item() < 1e-2
    finally:
        for h in hooks:
            h.remove()
    assert torch.equal(model(idx.to(dev), tg.to(dev), loss_reduction='none').cpu(), fused)  # fused again


def test_out_of_range_member_tables_give_nan_for_that_member_only(dev):
    """member_seq and member_row are read on the device. One member with member_row = n_rows and one with
    member_seq = -1 (passed past the host check): each gets a NaN loss (every token NaN), reads nothing out of range,
    and every other member's loss is bit-identical to the call with valid tables. The host check rejects both."""
    from noise_amd.population import Eggroll, NoiseLayout, run_forward
    print('population forward with out-of-range member tables m=6 T=256', flush=True)
    ocfg, gcfg = _cfgs()
    model = _model(dev, _weights(ocfg), gcfg)
    layout = NoiseLayout(model)
    es = Eggroll(model, 3, sigma=0.01, seed=5, chunk=3)
    rows = es.rows(es.offset_table(2), torch.arange(3, device=dev))
    idx, tg = recipe.tokens(ocfg, batch=2, seed=13)
    idx, tg = idx.to(dev), tg.to(dev)
    seq = torch.tensor([0, 1, 0, 1, 0, 1], dtype=torch.int32, device=dev)
    row = torch.tensor([0, 0, 1, 1, 2, 2], dtype=torch.int32, device=dev)
    sign = torch.tensor([0.01, -0.01] * 3, device=dev)
    good = run_forward(model, idx, tg, seq, noise=rows, member_row=row, member_sign=sign, layout=layout,
                       want_tokens=True)
    bad_seq, bad_row = seq.clone(), row.clone()
    bad_row[2] = 3          # one past the 3 noise rows
    bad_seq[5] = -1
    with pytest.raises(ValueError, match='member_row'):
        run_forward(model, idx, tg, seq, noise=rows, member_row=bad_row, member_sign=sign, layout=layout)
    with pytest.raises(ValueError, match='member_seq'):
        run_forward(model, idx, tg, bad_seq, noise=rows, member_row=row, member_sign=sign, layout=layout)
    out = run_forward(model, idx, tg, bad_seq, noise=rows, member_row=bad_row, member_sign=sign, layout=layout,
                      want_tokens=True, check_tables=False)
    loss, tok = out['loss_sum'].cpu(), out['token_loss'].cpu().view(6, -1)
    want, want_tok = good['loss_sum'].cpu(), good['token_loss'].cpu().view(6, -1)
    assert torch.isnan(loss[2]) and torch.isnan(loss[5]), loss
    assert torch.isnan(tok[2]).all() and torch.isnan(tok[5]).all()
    ok = [0, 1, 3, 4]
    assert torch.isfinite(want).all()
    assert torch.equal(loss[ok], want[ok]) and torch.equal(tok[ok], want_tok[ok])
