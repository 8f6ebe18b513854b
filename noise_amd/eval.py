"""The speedrun's score on this library's kernels: the mean next-token cross-entropy of a state dict over the fixed
validation rows, and the pinned token files it reads (interface of utils/eval.py:37-67 and
utils/prepare_data.py:20-48).

    python -m noise_amd.eval CHECKPOINT [--data-dir data]      # prints {"checkpoint": ..., "val_loss": ...}

Scoring: the checkpoint loads strictly into a fresh fixed-architecture GPT (a missing, extra or reshaped tensor is an
error). The rows then go through the population forward as unperturbed members, one member per row and up to
`batch_size` rows per launch sequence; each row's summed CE comes back separately and the total is kept in float64
on the device, divided by the number of predictions at the end. Under torch.distributed each rank takes a
contiguous share of the rows and the two sums are all-reduced. Only the fixed model is scored: a track 3 entry's
own model file (utils/eval.py:25-35) is another architecture and is refused.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
from pathlib import Path

import torch
from torch import distributed as dist

SEQ = 2049                # tokens per row, 2,048 predictions (utils/prepare_data.py:20)
TRAIN_ROWS = 14648        # utils/prepare_data.py:21
VAL_ROWS = 544            # utils/prepare_data.py:22
# sha256 over each split's tokens as int32 little-endian bytes (utils/prepare_data.py:27-30)
EXPECTED = {
    'train.pt': '2a92b8e9c3bc418c39880d337951775b9d29d0389bf1059cc826c412c44def37',
    'val.pt': '5fdb9242ce8ab83e519ab5dd5cf8d64f4d8a99f6e74c137f4ca0f723da5f7437',
}


def token_hash(rows: torch.Tensor) -> str:
    """Hex sha256 of the token values as int32 little-endian bytes, whatever the stored integer type."""
    data = rows.detach().to('cpu', torch.int32).contiguous().numpy().astype('<i4', copy=False)
    return hashlib.sha256(data.tobytes()).hexdigest()


def load_rows(path, rows: int) -> torch.Tensor:
    """The pinned split at `path` as int64 [rows, SEQ]: the file must hold a tensor of exactly this shape
    (ValueError), its name must be one of EXPECTED's (KeyError) and its token hash the pinned one (ValueError)."""
    path = Path(path)
    data = torch.load(path, map_location='cpu', weights_only=True)
    if not torch.is_tensor(data) or data.dim() != 2 or tuple(data.shape) != (rows, SEQ):
        raise ValueError(f'{path}: not a [{rows}, {SEQ}] token tensor')
    if token_hash(data) != EXPECTED[path.name]:
        raise ValueError(f'{path}: token hash mismatch (not the pinned data)')
    return data.to(torch.int64)


def load_model(state_dict, device, model_file=None, config=None):
    """A fresh fixed-architecture GPT on `device` holding exactly these weights, in eval mode without gradients."""
    from .model import GPT, GPTConfig
    if model_file is not None:
        raise ValueError('only the fixed model is scored here; a track 3 model file is another architecture')
    with torch.device('meta'):
        model = GPT(config or GPTConfig())
    model.to_empty(device=device)
    model.init_weights()
    model.load_state_dict(state_dict, strict=True)
    return model.eval().requires_grad_(False)


class Scorer:
    """Running float64 [summed CE, predictions] of rows scored on one model."""

    def __init__(self, model, batch_size=16):
        self.model, self.batch_size = model, batch_size
        self.device = model.lm_head.weight.device
        self.totals = torch.zeros(2, dtype=torch.float64, device=self.device)

    @torch.no_grad()
    def add(self, rows: torch.Tensor):
        from .population import run_forward
        for start in range(0, len(rows), self.batch_size):
            chunk = rows[start:start + self.batch_size].to(self.device, torch.int64)
            n = len(chunk)
            out = run_forward(self.model, chunk[:, :-1].contiguous(), chunk[:, 1:].contiguous(),
                              member_seq=torch.arange(n, dtype=torch.int32, device=self.device), check_tables=False)
            self.totals[0] += out['loss_sum'].double().sum()
            self.totals[1] += (chunk[:, 1:] >= 0).sum()

    def value(self) -> float:
        if dist.is_initialized() and dist.get_world_size() > 1:
            dist.all_reduce(self.totals)
        loss = (self.totals[0] / self.totals[1]).item()
        if not math.isfinite(loss):
            raise FloatingPointError(f'validation loss is not finite ({loss})')
        return loss


def _share(rows: torch.Tensor) -> torch.Tensor:
    """This rank's contiguous block of rows (all of them on one process)."""
    if not dist.is_initialized():
        return rows
    rank, world = dist.get_rank(), dist.get_world_size()
    bounds = [len(rows) * r // world for r in range(world + 1)]
    return rows[bounds[rank]:bounds[rank + 1]]


def evaluate(state_dict, data_dir='data', batch_size=16, model_file=None, *, rows=None, config=None):
    """Mean next-token CE of `state_dict` over the validation split of `data_dir` (or over `rows`, int64
    [n, T + 1], when given)."""
    device = torch.device('cuda', torch.cuda.current_device())
    model = load_model(state_dict, device, model_file, config)
    if rows is None:
        rows = load_rows(Path(data_dir) / 'val.pt', VAL_ROWS)
    T = rows.shape[1] - 1
    if T % 128:
        raise ValueError(f'rows of {T} predictions: the kernels take multiples of 128')
    scorer = Scorer(model, batch_size)
    scorer.add(_share(rows))
    return scorer.value()


def main():
    ap = argparse.ArgumentParser(prog='python -m noise_amd.eval', description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument('checkpoint', type=Path, help='state dict file written by a training run (final.pt)')
    ap.add_argument('--data-dir', type=Path, default=Path('data'), help='directory holding val.pt')
    args = ap.parse_args()
    world = int(os.environ.get('WORLD_SIZE', '1'))
    torch.cuda.set_device(int(os.environ.get('LOCAL_RANK', '0')))
    if world > 1:
        dist.init_process_group('nccl')
    try:
        state = torch.load(args.checkpoint, map_location='cpu', weights_only=True)
        loss = evaluate(state, args.data_dir)
        if not dist.is_initialized() or dist.get_rank() == 0:
            print(json.dumps({'checkpoint': str(args.checkpoint), 'val_loss': loss}), flush=True)
    finally:
        if dist.is_initialized():
            dist.destroy_process_group()


if __name__ == '__main__':
    main()
