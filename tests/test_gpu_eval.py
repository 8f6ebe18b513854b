"""The score path on the GPU (noise_amd/eval.py, utils/eval.py:48-66): evaluate() of a state dict saved and loaded
like a training script's final.pt, over token rows, against the fp32 oracle's mean next-token CE.

Tolerance 1e-2 relative: the forward's per-token loss bar (bf16 operands, fp32 accumulation)."""
import pytest
import torch

from oracle import model as om
from tests.golden import recipe

pytestmark = pytest.mark.gpu

SEQ = 256


def test_evaluate_matches_oracle(dev, tmp_path):
    print('evaluate: 5 rows of 257 tokens, batches of 2', flush=True)
    from noise_amd import eval as ne
    from noise_amd.model import GPTConfig
    ocfg = om.Config(sequence_len=SEQ)
    w = recipe.weights(ocfg, seed=99)
    for k in w:  # training keeps the embeddings in bf16 storage, so a checkpoint holds bf16 values
        if 'wte' in k or 'value_embeds' in k:
            w[k] = w[k].to(torch.bfloat16).float()
    torch.save(w, tmp_path / 'final.pt')
    sd = torch.load(tmp_path / 'final.pt', map_location='cpu', weights_only=True)
    idx, tg = recipe.tokens(ocfg, batch=5)
    rows = torch.cat([idx, tg[:, -1:]], dim=1)  # [5, 257]: inputs rows[:, :-1], targets rows[:, 1:]
    got = ne.evaluate(sd, rows=rows, config=GPTConfig(sequence_len=SEQ), batch_size=2)
    ref = om.gpt_forward(w, ocfg, idx, tg, 'sum').item() / tg.numel()
    assert abs(got - ref) / ref < 1e-2, (got, ref)
