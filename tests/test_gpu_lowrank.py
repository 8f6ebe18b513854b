"""GPU parity of the shared-x perturbed linear (config 2) against oracle.model.lowrank_sumsq.

Both evaluations of the per-member sums of squares (the expanded square on the MFMA units, and every element formed)
are checked against the float64 oracle. Tolerances: S_i within 1e-4 relative at the reduced shapes (bf16 operands,
fp32 accumulation; the roundings of x W^T and x . b agree with the oracle's except in rare last-bit ties); at the full
config-2 size the error must also stay within 1e-2 of S_i's member-specific part S_i - sum (x W^T)^2, which at
sigma 1e-3 is about 0.2% of S_i (so a wrong rank-1 term fails even though S_i barely moves)."""
import pytest
import torch

from oracle import model as om

pytestmark = pytest.mark.gpu


def _inputs(T, n_in, n_out, m, seed, a_off=7, gap=3):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, n_in, generator=g).bfloat16()
    W = (torch.randn(n_out, n_in, generator=g) * 0.02).bfloat16()
    stride = a_off + n_out + gap + n_in + 5
    rows = torch.randn(m, stride, generator=g)
    b_off = a_off + n_out + gap
    a, b = rows[:, a_off:a_off + n_out], rows[:, b_off:b_off + n_in]
    return x, W, rows, a_off, b_off, a, b


@pytest.mark.parametrize('mode', ['expansion', 'direct'])
def test_shared_sumsq_small(dev, mode):
    """m = 40 (a padded second member tile), 2 x 2 output tiles, sigma large enough that the rank-1 term dominates."""
    from noise_amd.population import lowrank_sumsq
    T, n_in, n_out, m = 512, 64, 512, 40
    print(f'lowrank shared {mode} T={T} in={n_in} out={n_out} m={m}', flush=True)
    x, W, rows, a_off, b_off, a, b = _inputs(T, n_in, n_out, m, seed=1)
    sign = torch.tensor([0.05 if i % 2 == 0 else -0.05 for i in range(m)])
    sign[5] = 0.0
    want, c2 = om.lowrank_sumsq(x.float(), W.float(), a, b, sign)
    got = lowrank_sumsq(x.to(dev), W.to(dev), rows.to(dev), a_off, b_off, sign.to(dev), mode=mode).cpu().double()
    rel = ((got - want).abs() / want.abs()).max().item()
    assert rel < 1e-4, rel
    assert abs(got[5] - c2) / c2 < 1e-5  # sign 0: the unperturbed sum of squares


def test_shared_modes_agree_and_y(dev):
    """With y stored, every element equals the oracle's c + (s u) a; the two evaluations give the same sums."""
    from noise_amd.population import lowrank, lowrank_sumsq
    T, n_in, n_out, m = 256, 96, 256, 3
    print(f'lowrank shared y T={T} in={n_in} out={n_out} m={m}', flush=True)
    x, W, rows, a_off, b_off, a, b = _inputs(T, n_in, n_out, m, seed=2)
    sign = torch.tensor([0.1, -0.1, 0.03])
    y = lowrank(x.to(dev), W.to(dev), a.to(dev), b.to(dev), sign.to(dev)).cpu().double()
    c = (x.float() @ W.float().t()).bfloat16().double()
    u = (x.float() @ b.bfloat16().float().t()).bfloat16().double()
    ref = c[None] + (sign.double()[:, None] * u.t())[:, :, None] * a.bfloat16().double()[:, None, :]
    # a last-bit tie of the bf16 rounding of x W^T or x . b may go the other way: one bf16 step of c or of the
    # rank-1 term at most, and only in rare elements (a tie in u moves one row of one member)
    err = (y - ref).abs()
    rank1 = ref - c[None]
    assert (err <= 2.0 ** -7 * (c.abs()[None] + rank1.abs()) + 1e-5).all(), err.max().item()
    assert (err > 1e-5).float().mean().item() < 2e-2
    s1 = lowrank_sumsq(x.to(dev), W.to(dev), rows.to(dev), a_off, b_off, sign.to(dev), mode='expansion').cpu()
    s2 = lowrank_sumsq(x.to(dev), W.to(dev), rows.to(dev), a_off, b_off, sign.to(dev), mode='direct').cpu()
    assert ((s1 - s2).abs() / s2.abs()).max().item() < 1e-5
    assert ((s2.double() - (y * y).sum((1, 2))).abs() / s2.double()).max().item() < 1e-5


def test_shared_gemm_is_the_same_bits_for_32_and_64_deep_k_steps(dev):
    """in = 512 takes the GEMM with 64-deep K steps (two LDS stages), in = 544 -- the same x and W with 32 zero
    columns appended -- the one with 32-deep steps (four stages): the same 16-deep MFMA products in the same order,
    plus exact zeros, so x W^T comes out with the same bits. (The signs are 0: the rank-1 term's x . b is summed by
    another kernel whose order depends on the width.)"""
    from noise_amd.population import lowrank
    T, n_in, n_out, m, pad = 512, 512, 512, 2, 32
    print(f'lowrank shared BK64 vs BK32 T={T} in={n_in}+{pad} out={n_out}', flush=True)
    x, W, rows, a_off, b_off, a, b = _inputs(T, n_in, n_out, m, seed=4)
    sign = torch.zeros(m)
    zx, zw = torch.zeros(T, pad, dtype=torch.bfloat16), torch.zeros(n_out, pad, dtype=torch.bfloat16)
    y64 = lowrank(x.to(dev), W.to(dev), a.to(dev), b.to(dev), sign.to(dev))
    y32 = lowrank(torch.cat([x, zx], 1).to(dev), torch.cat([W, zw], 1).to(dev), a.to(dev),
                  torch.cat([b, torch.zeros(m, pad)], 1).to(dev), sign.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(y64, y32)
    c = (x.float() @ W.float().t()).bfloat16()
    assert ((y64[0].float().cpu() - c.float()).abs() <= 2.0 ** -7 * c.float().abs() + 1e-6).all()


def test_shared_sumsq_config2(dev):
    """Config 2 at full size: X [32768, 512], W [2048, 512] N(0, 0.02), 64 members, sigma 1e-3; members 0 and 37
    against the float64 oracle, every member's two evaluations against each other."""
    from noise_amd.population import lowrank_sumsq
    T, n_in, n_out, m, sigma = 32768, 512, 2048, 64, 1e-3
    print(f'lowrank shared config 2 T={T} in={n_in} out={n_out} m={m}', flush=True)
    x, W, rows, a_off, b_off, a, b = _inputs(T, n_in, n_out, m, seed=3, a_off=0, gap=0)
    sign = torch.tensor([sigma if i % 2 == 0 else -sigma for i in range(m)])
    got = {md: lowrank_sumsq(x.to(dev), W.to(dev), rows.to(dev), a_off, b_off, sign.to(dev), mode=md).cpu().double()
           for md in ('expansion', 'direct')}
    assert ((got['expansion'] - got['direct']).abs() / got['direct']).max().item() < 1e-5
    pick = [0, 37]
    want, c2 = om.lowrank_sumsq(x.float(), W.float(), a, b, sign, members=pick)
    for md, s in got.items():
        for j, i in enumerate(pick):
            part = (want[j] - c2).abs().item()
            err = (s[i] - want[j]).abs().item()
            print(f'{md} member {i}: S {s[i].item():.6e} oracle {want[j].item():.6e} member part {part:.4e} '
                  f'err {err:.3e}', flush=True)
            assert err < 1e-3 * part, (md, i, err, part)  # measured 2.4e-5 of the member part
