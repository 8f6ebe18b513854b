"""GPU runs of the custom ops under torch.compile (fullgraph, the aot_eager backend: AOT tracing through the fake
kernels, no generated kernels): the compiled population_loss and lowrank equal the eager calls bit for bit and the
oracle within 1e-2 (per-member loss, relative). noise_linear against fp32 products of the same bf16 operands, and the
module-by-module (hooked) forward running its linears on it.

Tolerances: per-member losses 1e-2 relative (bf16 operands, fp32 accumulation); noise_linear within one bf16 rounding
of the fp32 product (2^-8 relative, plus 1e-6 absolute)."""
import pytest
import torch

from oracle import model as om
from tests.golden import recipe

pytestmark = pytest.mark.gpu


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


def test_compiled_population_loss_matches_eager_and_oracle(dev):
    from noise_amd.model import GPTConfig
    from noise_amd.population import population_loss
    print('torch.compile(population_loss) m=8 T=256', flush=True)
    torch._dynamo.reset()
    ocfg = om.Config(sequence_len=256)
    w = recipe.weights(ocfg, seed=99)
    model = _model(dev, w, GPTConfig(sequence_len=256))
    m, sigma = 8, 0.01
    noise = recipe.population_noise(ocfg, m, seed=21, step=3)
    sign = torch.tensor([sigma, -sigma] * (m // 2))
    idx, tg = recipe.tokens(ocfg, batch=1, seed=9)
    dnoise = {k: tuple(t.to(dev) for t in v) if isinstance(v, tuple) else v.to(dev) for k, v in noise.items()}
    args = (dnoise, sign.to(dev), idx[0].to(dev), tg[0].to(dev))
    params = dict(model.named_parameters())
    eager = population_loss(model, params, *args)
    compiled = torch.compile(population_loss, fullgraph=True, backend='aot_eager')
    got = compiled(model, params, *args)
    got2 = compiled(model, params, *args)  # a second call reuses the graph
    assert torch.equal(got, eager) and torch.equal(got2, eager)
    ref = om.population_loss(w, ocfg, noise, sign, idx[0], tg[0]) / ocfg.sequence_len
    rel = ((got.cpu() - ref).abs() / ref.abs()).max().item()
    print(f'compiled population_loss: max rel err vs oracle {rel:.3e}', flush=True)
    assert rel < 1e-2


def test_compiled_lowrank_matches_eager(dev):
    from noise_amd.population import lowrank, lowrank_embed
    print('torch.compile(lowrank / lowrank_embed)', flush=True)
    torch._dynamo.reset()
    g = torch.Generator(device=dev).manual_seed(5)
    m, T, n_in, n_out, V = 4, 256, 128, 512, 1000
    x = torch.randn(m, T, n_in, device=dev, generator=g).bfloat16()
    W = (torch.randn(n_out, n_in, device=dev, generator=g) * 0.05).bfloat16()
    a, b = torch.randn(m, n_out, device=dev, generator=g), torch.randn(m, n_in, device=dev, generator=g)
    sign = torch.tensor([0.01, -0.01, 0.02, -0.02], device=dev)
    f = torch.compile(lambda *t: lowrank(*t), fullgraph=True, backend='aot_eager')
    assert torch.equal(f(x, W, a, b, sign), lowrank(x, W, a, b, sign))
    E, ea = torch.randn(V, n_in, device=dev, generator=g), torch.randn(m, V, device=dev, generator=g)
    idx = torch.randint(0, V, (T,), device=dev, generator=g)
    fe = torch.compile(lambda *t: lowrank_embed(*t), fullgraph=True, backend='aot_eager')
    assert torch.equal(fe(E, ea, b, idx, sign), lowrank_embed(E, ea, b, idx, sign))


@pytest.mark.parametrize('M,n_in,n_out', [(4096, 512, 2048), (200, 512, 512), (1000, 2048, 512), (384, 512, 4096)])
def test_noise_linear_matches_fp32_product(dev, M, n_in, n_out):
    from noise_amd.model import linear_bf16
    print(f'noise_linear M={M} in={n_in} out={n_out}', flush=True)
    g = torch.Generator(device=dev).manual_seed(M + n_out)
    x = torch.randn(M, n_in, device=dev, generator=g).bfloat16()
    W = (torch.randn(n_out, n_in, device=dev, generator=g) * n_in ** -0.5).bfloat16()
    y = linear_bf16(x, W)
    ref = x.float() @ W.float().t()
    err = (y.float() - ref).abs()
    assert y.dtype == torch.bfloat16 and y.shape == (M, n_out)
    assert (err <= 2.0 ** -8 * ref.abs() + 1e-6).all(), err.max().item()
    # a strided row view: rows of a wider buffer
    wide = torch.zeros(M, n_in + 64, device=dev, dtype=torch.bfloat16)
    wide[:, :n_in] = x
    from noise_amd import _lib
    y2 = torch.empty_like(y)
    _lib.call('noise_linear', _lib.ptr(wide), n_in + 64, _lib.ptr(W), M, n_in, n_out, _lib.ptr(y2), n_out,
              _lib.stream(dev))
    assert torch.equal(y2, y)


def test_hooked_forward_runs_its_linears_on_noise_linear(dev):
    """A hooked GPT.forward (module by module) launches noise_linear for c_q, c_k, c_v, c_proj, c_fc, mlp c_proj and
    lm_head: 6 per block plus the head."""
    from noise_amd import _lib
    from noise_amd.model import GPTConfig
    print('hooked forward on noise_linear B=2 T=256', flush=True)
    ocfg = om.Config(sequence_len=256)
    w = recipe.weights(ocfg, seed=99)
    model = _model(dev, w, GPTConfig(sequence_len=256))
    idx, tg = recipe.tokens(ocfg, batch=2, seed=51)
    h = model.lm_head.register_forward_hook(lambda *a: None)
    try:
        torch.cuda.synchronize()
        _lib.timing_enable(True)
        with torch.no_grad():
            got = model(idx.to(dev), tg.to(dev), loss_reduction='none').cpu()
        tm = _lib.timing_read()
        _lib.timing_enable(False)
    finally:
        h.remove()
    assert tm['linear'][0] == 6 * ocfg.n_layer + 1, tm.get('linear')
    ref = om.gpt_forward(w, ocfg, idx, tg, 'none')
    assert ((got - ref).abs() / ref.abs()).max().item() < 1e-2
