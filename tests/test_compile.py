"""The population forward, lowrank and lowrank_embed as torch.library custom ops with fake kernels: a compiled caller
(the reference compiles population_loss, archive/10M/train/val/eggroll.py:115) traces each into ONE graph with the
op inside, no graph break. Traced on the CPU with fake tensors (the backend records the graph and runs nothing); the
GPU tests run the compiled functions against the oracle."""
import pytest
import torch

from oracle import model as om
from tests.golden import recipe


def _recording_backend(graphs, out):
    def backend(gm, example_inputs):
        graphs.append(gm)
        return lambda *args: out
    return backend


def _cpu_model(n_layer=2, T=256):
    from noise_amd.model import GPT, GPTConfig
    torch.manual_seed(0)
    model = GPT(GPTConfig(n_layer=n_layer, sequence_len=T))
    model.init_weights()
    return model


def _ops(gm):
    return {str(n.target) for n in gm.graph.nodes if n.op == 'call_function'}


def test_population_loss_traces_into_one_graph():
    from noise_amd.population import population_loss
    torch._dynamo.reset()
    model = _cpu_model()
    ocfg = om.Config(n_layer=2, sequence_len=256)
    m = 4
    noise = recipe.population_noise(ocfg, m, seed=3, step=1)
    sign = torch.tensor([0.01, -0.01] * (m // 2))
    idx, tg = recipe.tokens(ocfg, batch=1, seed=5)
    graphs = []
    fn = torch.compile(population_loss, fullgraph=True, backend=_recording_backend(graphs, (torch.zeros(m),)))
    fn(model, dict(model.named_parameters()), noise, sign, idx[0], tg[0])
    assert len(graphs) == 1
    ops = _ops(graphs[0])
    assert 'noise_amd.population_forward' in ops, ops
    # p = None (the model's own parameters) traces too
    torch._dynamo.reset()
    graphs.clear()
    fn = torch.compile(population_loss, fullgraph=True, backend=_recording_backend(graphs, (torch.zeros(m),)))
    fn(model, None, noise, sign, idx[0], tg[0])
    assert len(graphs) == 1


def test_lowrank_ops_trace_into_one_graph():
    from noise_amd.population import lowrank, lowrank_embed
    torch._dynamo.reset()
    m, T, n_in, n_out, V = 3, 128, 64, 256, 300
    x = torch.randn(m, T, n_in)
    W = torch.randn(n_out, n_in)
    a, b, sign = torch.randn(m, n_out), torch.randn(m, n_in), torch.randn(m)
    graphs = []
    fn = torch.compile(lambda *t: lowrank(*t) * 2, fullgraph=True,
                       backend=_recording_backend(graphs, (torch.zeros(m, T, n_out),)))
    fn(x, W, a, b, sign)
    assert len(graphs) == 1 and 'noise_amd.lowrank' in _ops(graphs[0])
    torch._dynamo.reset()
    graphs.clear()
    E, ea = torch.randn(V, n_in), torch.randn(m, V)
    idx = torch.randint(0, V, (T,))
    fn = torch.compile(lambda *t: lowrank_embed(*t) + 1, fullgraph=True,
                       backend=_recording_backend(graphs, (torch.zeros(m, T, n_in),)))
    fn(E, ea, b, idx, sign)
    assert len(graphs) == 1 and 'noise_amd.lowrank_embed' in _ops(graphs[0])


def test_fake_kernels_give_the_real_shapes():
    """The fake kernels' outputs, which a compiled caller's later ops are traced against."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x, W = torch.empty(4, 128, 64), torch.empty(256, 64)
        y = torch.ops.noise_amd.lowrank(x, W, torch.empty(4, 256), torch.empty(4, 64), torch.empty(4))
        assert y.shape == (4, 128, 256) and y.dtype == torch.float32
        e = torch.ops.noise_amd.lowrank_embed(torch.empty(300, 64), torch.empty(4, 300), torch.empty(4, 64),
                                              torch.empty(128, dtype=torch.int64), torch.empty(4))
        assert e.shape == (4, 128, 64) and e.dtype == torch.float32
