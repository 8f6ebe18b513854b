"""Write the golden fixtures of tests/golden/ from the reference's own Python functions.

Runs only where the reference checkout is mounted (never on the GPU box, never at test time):
    python tests/golden/make_golden.py [/root/reference]

What is imported from the reference, and why (only what no closed form pins):
  utils/model.py GPT.forward (:193-210)     the composite numerics: rms_norm eps, bf16 rotary tables, window masks,
                                            softcap, ignore_index, op order
  utils/model.py GPT named_parameters       the parameter order the noise offsets are keyed by
  archive/10M/train/val/eggroll.py population_loss (:66-103)   the perturbed forward end to end
The compiled flex kernel (utils/model.py:14) does not build on CPU here (Inductor IndexError), so the reference
module's `flex` is replaced by torch's eager flex_attention, the same function unfused. Everything runs in fp32 on
CPU without autocast. Inputs (weights, tokens, noise) come from tests/golden/recipe.py; the fixtures hold outputs.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle.model import Config  # noqa: E402
from tests.golden import recipe  # noqa: E402


def main(ref_root='/root/reference'):
    sys.path.insert(0, ref_root)
    sys.path.insert(0, str(Path(ref_root) / 'archive' / '10M' / 'train' / 'val'))
    import utils.model as um
    from torch.nn.attention.flex_attention import flex_attention
    um.flex = flex_attention
    import eggroll as eg
    eg.attention = um.attention

    # parameter order of the default model (no compute: meta device)
    with torch.device('meta'):
        full = um.GPT(um.GPTConfig())
    order = [[n, list(p.shape)] for n, p in full.named_parameters()]
    (HERE / 'param_order.json').write_text(json.dumps(order, indent=0) + '\n')

    cfg = Config(**recipe.SMALL)
    ucfg = um.GPTConfig(**recipe.SMALL)
    with torch.device('meta'):
        model = um.GPT(ucfg)
    model.to_empty(device='cpu')
    model.init_weights()
    w = recipe.weights(cfg)
    model.load_state_dict(w, strict=True)
    model.requires_grad_(False)

    idx, targets = recipe.tokens(cfg, batch=2, ignore_every=29)
    with torch.no_grad():
        ce = model(idx, targets, loss_reduction='none')
        logits = model(idx)
    np.savez(HERE / 'gpt_forward_small.npz', ce=ce.numpy().astype(np.float32),
             logits_b0=logits[0, [0, 31, 63]].numpy().astype(np.float32))

    members, sigma = 4, 0.05
    noise = recipe.population_noise(cfg, members)
    sign = torch.tensor([sigma, -sigma] * (members // 2))
    p = dict(model.named_parameters())
    idx1, targets1 = recipe.tokens(cfg, batch=1, seed=recipe.TOKEN_SEED + 1)
    with torch.no_grad():
        mean_ce = eg.population_loss(model, p, noise, sign, idx1[0], targets1[0])
    np.savez(HERE / 'population_loss_small.npz', mean_ce=mean_ce.numpy().astype(np.float32),
             sigma=np.float32(sigma))
    print('param_order', len(order), 'ce', ce[:4].tolist(), 'population', mean_ce.tolist())


if __name__ == '__main__':
    main(*sys.argv[1:])
