"""The EGGROLL training run (archive/10M/train/val/eggroll.py:171-250) on this library's population step.

    python -m noise_amd.train [--data-dir data] [--output logs/eggroll] [--steps K] [--eval-every E] [--pairs P] [--lr LR]

One epoch: the training rows, shuffled by seed + 1, feed BATCH sequences per update. An untimed warmup update on random
tokens runs first; model, optimizer and population are then rebuilt from the seed, so the timed run starts as if the
warmup had not happened. Every update sets the warmdown learning rate, runs Eggroll.step and appends
{step, population_loss, train_seconds[, val_loss]} to metrics.jsonl (untimed validation every --eval-every updates);
the end writes final.pt (the state dict) and result.json {val_loss, train_seconds, steps, tokens}. Under torchrun every
rank evaluates its share of the members and rank 0 writes the files, as the reference does.
"""
from __future__ import annotations

import argparse
import json
import os
import time
from pathlib import Path

import torch
from torch import distributed as dist

from .eval import TRAIN_ROWS, evaluate, load_rows
from .model import GPT, GPTConfig
from .optim import AdamW
from .population import CHUNK, SEED, SIGMA, Eggroll

BATCH = 8            # sequences per update (eggroll.py:28)
PAIRS = 131072       # antithetic pairs per update (eggroll.py:30)
LR, BETAS = 0.001, (0.5, 0.95)
WARMDOWN = 0.3       # final fraction of the epoch over which the learning rate decays linearly to 0


def make_model(device, seed=SEED):
    """eggroll.py:38-52: the fixed model's initialization, c_proj weights U(+-1.5 sqrt(3 / in)), and the embeddings
    kept in float32 for the updates."""
    torch.manual_seed(seed)
    with torch.device('meta'):
        model = GPT(GPTConfig())
    model.to_empty(device=device)
    model.init_weights()
    with torch.no_grad():
        for name, module in model.named_modules():
            if 'c_proj' in name and isinstance(module, torch.nn.Linear):
                scale = 1.5 * (3 / module.weight.shape[1]) ** 0.5
                torch.nn.init.uniform_(module.weight, -scale, scale)
    model.transformer.wte.float()
    for embedding in model.value_embeds.values():
        embedding.float()
    return model.requires_grad_(False)


def train(data_dir='data', output='logs/eggroll', steps=None, eval_every=0, pairs=PAIRS, lr=LR, *, rows=None,
          val_rows=None, log=print):
    """The run of eggroll.py:main. `rows` (int64 [n, 2049]) and `val_rows` replace the pinned token files when given.
    Returns the result dict (rank 0) or None."""
    rank, world = (dist.get_rank(), dist.get_world_size()) if dist.is_initialized() else (0, 1)
    if (2 * pairs) % (world * 2 * CHUNK):
        raise ValueError('Each GPU must evaluate whole chunks of pairs.')
    output = Path(output)
    training = load_rows(Path(data_dir) / 'train.pt', TRAIN_ROWS) if rows is None else rows.long()
    training = training[torch.randperm(len(training), generator=torch.Generator().manual_seed(SEED + 1))]
    steps = min(len(training) // BATCH, steps or len(training))
    if steps < 1:
        raise ValueError(f'{len(training)} rows make no update of {BATCH} sequences')
    device = torch.device('cuda', torch.cuda.current_device())
    if rank == 0:
        if output.exists() and any(output.iterdir()):
            raise FileExistsError(f'Choose an empty output directory: {output}')
        output.mkdir(parents=True, exist_ok=True)
        (output / 'config.json').write_text(json.dumps(dict(
            script='noise_amd/train.py', world=world, batch=BATCH, steps=steps, seed=SEED, pairs=pairs, sigma=SIGMA,
            lr=lr, betas=BETAS, warmdown=WARMDOWN, torch_version=torch.__version__,
        ), indent=2) + '\n')

    def init():
        model = make_model(device, SEED)
        optimizer = AdamW(model.parameters(), lr=lr, betas=BETAS, eps=1e-8, weight_decay=0.0)
        return model, optimizer, Eggroll(model, pairs, rank, world)

    def set_rate(optimizer, step):
        left = (steps - step + 1) / steps  # fraction of the epoch still ahead, this update included
        for group in optimizer.param_groups:
            group.setdefault('initial_lr', group['lr'])
            group['lr'] = group['initial_lr'] * min(1.0, left / WARMDOWN)

    evaluate_kw = dict(data_dir=data_dir, rows=val_rows)
    model, optimizer, es = init()
    noise = torch.randint(0, 4096, (BATCH, 2049), generator=torch.Generator().manual_seed(SEED)).to(device)
    es.step(noise[:, :-1].contiguous(), noise[:, 1:].contiguous(), optimizer, 0)
    model, optimizer, es = init()

    if rank == 0:
        log(f'eggroll: {steps} steps, {pairs} pairs, sigma={SIGMA}, lr={lr}, GPUs={world}')
    metrics = (output / 'metrics.jsonl').open('a') if rank == 0 else None
    torch.cuda.synchronize()
    start, paused, elapsed = time.perf_counter(), 0.0, 0.0
    step = 0
    try:
        for step in range(1, steps + 1):
            batch = training[(step - 1) * BATCH:step * BATCH].to(device)
            set_rate(optimizer, step)
            loss = es.step(batch[:, :-1].contiguous(), batch[:, 1:].contiguous(), optimizer, step)
            torch.cuda.synchronize()
            elapsed = time.perf_counter() - start - paused
            record = dict(step=step, population_loss=loss, train_seconds=round(elapsed, 2))
            if eval_every and step % eval_every == 0 and step < steps:
                pause = time.perf_counter()
                record['val_loss'] = evaluate(model.state_dict(), **evaluate_kw)
                paused += time.perf_counter() - pause
            if rank == 0:
                log(json.dumps(record))
                metrics.write(json.dumps(record) + '\n')
                metrics.flush()
    finally:
        if metrics:
            metrics.close()

    state = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    val_loss = evaluate(state, **evaluate_kw)
    if rank != 0:
        return None
    torch.save(state, output / 'final.pt')
    result = dict(val_loss=val_loss, train_seconds=round(elapsed, 2), steps=step, tokens=step * BATCH * 2048)
    (output / 'result.json').write_text(json.dumps(result, indent=2) + '\n')
    log(json.dumps(result))
    return result


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument('--data-dir', type=Path, default=Path('data'))
    parser.add_argument('--output', type=Path, default=Path('logs/eggroll'))
    parser.add_argument('--steps', type=int, help='Stop after this many updates (smoke tests).')
    parser.add_argument('--eval-every', type=int, default=0, help='Untimed validation every this many updates.')
    parser.add_argument('--pairs', type=int, default=PAIRS, help='Antithetic pairs per update.')
    parser.add_argument('--lr', type=float, default=LR, help='Adam learning rate.')
    args = parser.parse_args()
    world = int(os.environ.get('WORLD_SIZE', 1))
    torch.cuda.set_device(int(os.environ.get('LOCAL_RANK', 0)))
    if world > 1:
        dist.init_process_group('nccl')
    try:
        train(args.data_dir, args.output, args.steps, args.eval_every, args.pairs, args.lr,
              log=lambda s: print(s, flush=True))
    finally:
        if world > 1:
            dist.destroy_process_group()


if __name__ == '__main__':
    main()
