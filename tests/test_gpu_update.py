"""GPU parity of the EGGROLL update (fitness, gradients, AdamW) and of a whole Eggroll.step against the oracle.

Tolerances: fitness and AdamW fp32 (1e-5 relative); gradients assembled in fp32 from the same noise (1e-4 relative);
per-member losses 1e-2 relative (bf16 forward)."""
import numpy as np
import pytest
import torch

from oracle import eggroll as oe
from oracle import model as om
from tests.golden import recipe

pytestmark = pytest.mark.gpu


def test_fitness(dev):
    from noise_amd import _lib
    r = np.random.default_rng(0)
    for members, pairs in [(64, 32), (24576, 12288), (48, 8)]:
        L = torch.from_numpy(r.normal(8.3, 0.05, members).astype(np.float32))
        f = torch.empty(members // 2, device=dev)
        w = torch.empty(pairs, device=dev)
        L_d = L.to(dev)
        _lib.call('noise_fitness', _lib.ptr(L_d), members, pairs, _lib.ptr(f), _lib.ptr(w), _lib.stream(dev))
        fr = oe.fitness(L)
        wr = oe.direction_weights(fr, pairs)
        assert torch.allclose(f.cpu(), fr, rtol=1e-4, atol=1e-4)
        assert torch.allclose(w.cpu(), wr, rtol=1e-4, atol=1e-4)


def test_outer_grad_and_vector_grad(dev):
    from noise_amd import _lib
    g = torch.Generator().manual_seed(1)
    pairs, out, n_in, stride = 300, 130, 70, 260
    rows = torch.randn(pairs, stride, generator=g)
    w = torch.randn(pairs, generator=g)
    grad = torch.empty(out, n_in, device=dev)
    rows_d, w_d = rows.to(dev), w.to(dev)  # held: a freed temporary's block could be reused before the launch
    _lib.call('noise_outer_grad', _lib.ptr(rows_d), stride, 5, 5 + out, _lib.ptr(w_d), pairs, out, n_in,
              -0.25, 0, _lib.ptr(grad), _lib.stream(dev))
    want = -0.25 * (w[:, None] * rows[:, 5:5 + out]).t().double() @ rows[:, 5 + out:5 + out + n_in].double()
    assert torch.allclose(grad.cpu().double(), want, rtol=1e-4, atol=1e-4)
    vec = torch.empty(8, device=dev)
    _lib.call('noise_outer_grad', _lib.ptr(rows_d), stride, 3, -1, _lib.ptr(w_d), pairs, 1, 8, 2.0, 0,
              _lib.ptr(vec), _lib.stream(dev))
    assert torch.allclose(vec.cpu(), 2.0 * (w @ rows[:, 3:11]), rtol=1e-4, atol=1e-4)
    vec21 = torch.empty(21, device=dev)  # three 8-element blocks, the last partial
    _lib.call('noise_outer_grad', _lib.ptr(rows_d), stride, 17, -1, _lib.ptr(w_d), pairs, 1, 21, -1.5, 0,
              _lib.ptr(vec21), _lib.stream(dev))
    assert torch.allclose(vec21.cpu(), -1.5 * (w @ rows[:, 17:38]), rtol=1e-4, atol=1e-4)
    # accumulate: the pairs in two chunks, the second added to the first
    half = pairs // 2
    acc = torch.empty(out, n_in, device=dev)
    vacc = torch.empty(21, device=dev)
    for k, (lo, hi) in enumerate([(0, half), (half, pairs)]):
        r, ww = rows_d[lo:hi].contiguous(), w_d[lo:hi].contiguous()
        _lib.call('noise_outer_grad', _lib.ptr(r), stride, 5, 5 + out, _lib.ptr(ww), hi - lo, out, n_in, -0.25, k,
                  _lib.ptr(acc), _lib.stream(dev))
        _lib.call('noise_outer_grad', _lib.ptr(r), stride, 17, -1, _lib.ptr(ww), hi - lo, 1, 21, -1.5, k,
                  _lib.ptr(vacc), _lib.stream(dev))
    torch.cuda.synchronize()
    assert torch.allclose(acc.cpu().double(), want, rtol=1e-4, atol=1e-4)
    assert torch.allclose(vacc.cpu(), -1.5 * (w @ rows[:, 17:38]), rtol=1e-4, atol=1e-4)


def test_outer_grad_batch(dev):
    """Several matrices in one grouped launch: unaligned slice offsets, sizes that are not multiples of the 128 x 128
    tile or of 4, a pair count that is not a multiple of the 16-pair stage, a matrix smaller than one tile and one
    spanning many; each against its float64 outer-product sum."""
    from noise_amd import _lib
    import ctypes
    g = torch.Generator().manual_seed(3)
    pairs, stride = 333, 2100
    rows = torch.randn(pairs, stride, generator=g)
    w = torch.randn(pairs, generator=g)
    mats = [(5, 300, 8, 32), (41, 700, 130, 70), (1, 2, 512, 513), (777, 1290, 257, 129)]  # a_off, b_off, out, in
    grads = [torch.full((o, i), float('nan'), device=dev) for _, _, o, i in mats]
    rows_d, w_d = rows.to(dev), w.to(dev)
    arr = lambda vals, t: (t * len(vals))(*vals)
    _lib.call('noise_outer_grad_batch', _lib.ptr(rows_d), stride, _lib.ptr(w_d), pairs, len(mats),
              arr([m[0] for m in mats], ctypes.c_int64), arr([m[1] for m in mats], ctypes.c_int64),
              arr([m[2] for m in mats], ctypes.c_int64), arr([m[3] for m in mats], ctypes.c_int64),
              arr([t.data_ptr() for t in grads], ctypes.c_void_p), 0.5, 0, _lib.stream(dev))
    for (a0, b0, o, i), got in zip(mats, grads):
        want = 0.5 * (w[:, None] * rows[:, a0:a0 + o]).t().double() @ rows[:, b0:b0 + i].double()
        assert torch.allclose(got.cpu().double(), want, rtol=1e-4, atol=1e-4), (o, i)


def test_outer_grad_batch_over_several_launches(dev):
    """70 small matrices: more than one launch's 64-job table, so the entry point splits the list."""
    from noise_amd import _lib
    import ctypes
    g = torch.Generator().manual_seed(4)
    pairs, stride = 40, 400
    rows = torch.randn(pairs, stride, generator=g)
    w = torch.randn(pairs, generator=g)
    mats = [(k, 200 + 2 * k, 3 + k % 5, 1 + k % 7) for k in range(70)]
    grads = [torch.full((o, i), float('nan'), device=dev) for _, _, o, i in mats]
    rows_d, w_d = rows.to(dev), w.to(dev)
    arr = lambda vals, t: (t * len(vals))(*vals)
    _lib.call('noise_outer_grad_batch', _lib.ptr(rows_d), stride, _lib.ptr(w_d), pairs, len(mats),
              arr([m[0] for m in mats], ctypes.c_int64), arr([m[1] for m in mats], ctypes.c_int64),
              arr([m[2] for m in mats], ctypes.c_int64), arr([m[3] for m in mats], ctypes.c_int64),
              arr([t.data_ptr() for t in grads], ctypes.c_void_p), 1.0, 0, _lib.stream(dev))
    for (a0, b0, o, i), got in zip(mats, grads):
        want = (w[:, None] * rows[:, a0:a0 + o]).t().double() @ rows[:, b0:b0 + i].double()
        assert torch.allclose(got.cpu().double(), want, rtol=1e-4, atol=1e-4), (a0, o, i)


def test_adamw_matches_torch(dev):
    from noise_amd.optim import AdamW
    g = torch.Generator().manual_seed(2)
    p0 = torch.randn(5000, generator=g)
    ref = torch.nn.Parameter(p0.clone())
    mine = torch.nn.Parameter(p0.clone().to(dev))
    opt_ref = torch.optim.AdamW([ref], lr=1e-3, betas=(0.5, 0.95), eps=1e-8, weight_decay=0.0)
    opt = AdamW([mine], lr=1e-3, betas=(0.5, 0.95), eps=1e-8, weight_decay=0.0)
    for _ in range(4):
        grad = torch.randn(5000, generator=g)
        ref.grad, mine.grad = grad.clone(), grad.to(dev)
        opt_ref.step()
        opt.step()
    assert torch.allclose(mine.detach().cpu(), ref.detach(), rtol=1e-5, atol=1e-7)


def test_adamw_groups_weight_decay_and_skipped_steps_match_torch(dev):
    """Two groups, one with weight decay 0.1; ragged sizes (the 4-wide vector path and its tail); one parameter gets
    no gradient at step 2, so its moments run one step behind the others of its group (a separate launch)."""
    from noise_amd.optim import AdamW
    g = torch.Generator().manual_seed(5)
    sizes = [[5001, 64, 7], [4096, 3]]
    init = [[torch.randn(n, generator=g) for n in grp] for grp in sizes]
    ref = [[torch.nn.Parameter(t.clone()) for t in grp] for grp in init]
    mine = [[torch.nn.Parameter(t.clone().to(dev)) for t in grp] for grp in init]
    conf = [dict(lr=1e-3, weight_decay=0.1), dict(lr=3e-2, weight_decay=0.0)]
    opt_ref = torch.optim.AdamW([dict(params=p, **c) for p, c in zip(ref, conf)], betas=(0.7, 0.95), eps=1e-8)
    opt = AdamW([dict(params=p, **c) for p, c in zip(mine, conf)], betas=(0.7, 0.95), eps=1e-8)
    for step in range(4):
        for gi, grp in enumerate(sizes):
            for pi, n in enumerate(grp):
                skip = step == 1 and (gi, pi) == (0, 1)
                grad = None if skip else torch.randn(n, generator=g)
                ref[gi][pi].grad = None if skip else grad.clone()
                mine[gi][pi].grad = None if skip else grad.to(dev)
        opt_ref.step()
        opt.step()
    for gi, grp in enumerate(sizes):
        for pi in range(len(grp)):
            assert torch.allclose(mine[gi][pi].detach().cpu(), ref[gi][pi].detach(), rtol=1e-5, atol=1e-7), (gi, pi)
    assert opt.state[mine[0][1]]['step'] == 3 and opt.state[mine[0][0]]['step'] == 4


def test_adamw_batch_many_tensors_with_empty_ones_match_torch(dev):
    """More tensors than one launch takes (48), with empty tensors among them (two inside the first 48, one at the
    start of the second launch's range, one last): every tensor must take exactly one step per call, so the result
    equals torch.optim.AdamW after 3 steps. A tensor stepped twice (the batching's cursor restarting behind the last
    tensor it took) would differ by a whole Adam step."""
    from noise_amd.optim import AdamW
    g = torch.Generator().manual_seed(11)
    sizes = [int(s) for s in torch.randint(1, 300, (60,), generator=g)]
    for j in (3, 20, 48, 59):
        sizes[j] = 0
    init = [torch.randn(n, generator=g) for n in sizes]
    ref = [torch.nn.Parameter(t.clone()) for t in init]
    mine = [torch.nn.Parameter(t.clone().to(dev)) for t in init]
    opt_ref = torch.optim.AdamW(ref, lr=1e-2, betas=(0.8, 0.95), eps=1e-8, weight_decay=0.1)
    opt = AdamW(mine, lr=1e-2, betas=(0.8, 0.95), eps=1e-8, weight_decay=0.1)
    for _ in range(3):
        for r, m, n in zip(ref, mine, sizes):
            grad = torch.randn(n, generator=g)
            r.grad, m.grad = grad.clone(), grad.to(dev)
        opt_ref.step()
        opt.step()
    for j, (r, m) in enumerate(zip(ref, mine)):
        assert torch.allclose(m.detach().cpu(), r.detach(), rtol=1e-5, atol=1e-7), (j, sizes[j])


def test_eggroll_step_decomposed(dev):
    """One Eggroll.step on a 256-token model: losses vs the oracle's population forward, fitness from those losses,
    and the gradient the oracle assembles from the GPU's own direction weights."""
    from noise_amd.model import GPT, GPTConfig
    from noise_amd.population import Eggroll
    ocfg = om.Config(sequence_len=256)
    w = recipe.weights(ocfg, seed=99)
    with torch.device('meta'):
        model = GPT(GPTConfig(sequence_len=256))
    model.to_empty(device=dev)
    model.init_weights()
    model.transformer.wte.float()
    for e in model.value_embeds.values():
        e.float()
    model.load_state_dict({k: v.to(dev) for k, v in w.items()}, strict=True)
    model.requires_grad_(False)
    pairs, sigma, seed, step = 8, 0.05, 3, 1
    es = Eggroll(model, pairs, sigma=sigma, seed=seed, chunk=4)
    idx, tg = recipe.tokens(ocfg, batch=2, seed=41)
    opt = torch.optim.SGD(model.parameters(), lr=0.0)  # the step's own optimizer call; lr 0 keeps the weights
    es.step(idx.to(dev), tg.to(dev), opt, step)
    losses = es.last['losses'].cpu()
    grads = {n: p.grad.detach().cpu() for n, p in model.named_parameters()}

    d, s, q = oe.member_layout(pairs, 2, chunk=4)
    offs = oe.step_offsets(ocfg, seed, step, pairs)
    ref = torch.empty(len(d))
    for seq in range(2):
        sel = np.nonzero(q == seq)[0]
        noise = oe.noise(ocfg, seed, offs, d[sel])
        ref[sel] = om.population_loss(w, ocfg, noise, torch.tensor(s[sel] * sigma, dtype=torch.float32),
                                      idx[seq], tg[seq]) / 256
    assert ((losses - ref).abs() / ref).max().item() < 1e-2
    weight = es.last['weight'].cpu()
    assert torch.allclose(es.last['fitness'].cpu(), oe.fitness(losses), rtol=1e-4, atol=1e-4)
    want = oe.gradients(ocfg, seed, offs, weight, n_fitness=len(d) // 2)
    for name, gv in want.items():
        err = (grads[name] - gv).abs().max().item() / max(gv.abs().max().item(), 1e-12)
        assert err < 1e-4, (name, err)
