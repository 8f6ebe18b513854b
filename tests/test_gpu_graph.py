"""HIP-graph capture of the boundary's ops (the reference replays whole steps as CUDA graphs,
train/speedrun/run.py:4062-4064, 4105-4107): one population forward with noise plus one credit readout, captured
after a warm-up with timing off, replays bit for bit equal to the eager calls, several times, with eager work and
synchronizations between the replays (nothing in these paths records a memset, allocates or synchronizes)."""
import pytest
import torch

from oracle import model as om
from tests.golden import recipe

pytestmark = pytest.mark.gpu


def test_population_forward_and_credit_replay_bit_for_bit(dev):
    from noise_amd import _lib, credit
    from noise_amd.model import GPT, GPTConfig
    from noise_amd.population import Eggroll, NoiseLayout, run_forward
    print('graph capture: population forward m=8 T=256 + credit readout', flush=True)
    _lib.timing_enable(False)
    ocfg = om.Config(sequence_len=256)
    w = recipe.weights(ocfg, seed=21)
    with torch.device('meta'):
        model = GPT(GPTConfig(sequence_len=256))
    model.to_empty(device=dev)
    model.init_weights()
    model.transformer.wte.float()
    for e in model.value_embeds.values():
        e.float()
    model.load_state_dict({k: v.to(dev) for k, v in w.items()}, strict=True)
    layout = NoiseLayout(model)
    es = Eggroll(model, 4, sigma=0.01, seed=3, chunk=4)
    rows = es.rows(es.offset_table(1), torch.arange(4, device=dev))
    idx, tg = recipe.tokens(ocfg, batch=2, seed=61)
    idx, tg = idx.to(dev), tg.to(dev)
    member_seq = torch.tensor([0, 1] * 4, dtype=torch.int32, device=dev)
    member_row = torch.tensor([0, 0, 1, 1, 2, 2, 3, 3], dtype=torch.int32, device=dev)
    member_sign = torch.tensor([0.01, -0.01] * 4, device=dev)
    g = torch.Generator(device=dev).manual_seed(4)
    q = (torch.randn(16, 256, 64, device=dev, generator=g) / 8).bfloat16()
    k = (torch.randn(16, 256, 64, device=dev, generator=g) / 8).bfloat16()
    e = torch.randn(16, 256, 64, device=dev, generator=g)

    def work():
        out = run_forward(model, idx, tg, member_seq, noise=rows, member_row=member_row, member_sign=member_sign,
                          layout=layout, want_tokens=True, check_tables=False)  # no host sync under capture
        return out['loss_sum'], out['token_loss'], credit.value_credit(q, k, e, 128)

    eager = [t.clone() for t in work()]
    for _ in range(2):
        work()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = work()
    for rep in range(3):
        for t in captured:
            t.fill_(float('nan'))
        graph.replay()
        torch.cuda.synchronize()
        for want, got in zip(eager, captured):
            assert torch.equal(got, want), (rep, (got - want).abs().max().item())
        again = work()  # eager work on the same workspace between replays
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(again, eager))
    assert torch.isfinite(eager[0]).all() and eager[0].std() > 0
