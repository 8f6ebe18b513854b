"""The speedrun's score on the HIP forward: mean next-token cross-entropy of a state dict over the fixed validation
rows (utils/eval.py), with the pinned token files of utils/prepare_data.py:20-48.

    python -m noise_amd.eval logs/val/final.pt [--data-dir data]

The weights load strictly into a fresh noise_amd GPT (the reference's names, shapes and order), built on the meta
device and materialized on the GPU as utils/eval.py:38-45 does; every batch then runs the population forward's
kernels with no noise (one evaluation per row), summing the per-token CE exactly as GPT.forward(...,
loss_reduction='sum') does under bf16 autocast. Only the fixed model is supported: track 3's own model files
(utils/eval.py:25-35) are another architecture.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
from pathlib import Path

import torch
from torch import distributed as dist

SEQ = 2049                # tokens per row: 2,048 predictions (utils/prepare_data.py:20)
TRAIN_ROWS = 14648        # 29,999,104 prediction tokens
VAL_ROWS = 544            # 1,114,112 prediction tokens
# sha256 of each split's int32 little-endian token bytes, independent of the torch.save container
# (utils/prepare_data.py:27-30): the data is pinned by these values
EXPECTED = {
    'train.pt': '2a92b8e9c3bc418c39880d337951775b9d29d0389bf1059cc826c412c44def37',
    'val.pt': '5fdb9242ce8ab83e519ab5dd5cf8d64f4d8a99f6e74c137f4ca0f723da5f7437',
}


def token_hash(rows: torch.Tensor) -> str:
    """sha256 of the rows as int32 little-endian bytes (utils/prepare_data.py:36-37)."""
    return hashlib.sha256(rows.to(torch.int32).contiguous().numpy().astype('<i4').tobytes()).hexdigest()


def load_rows(path, rows: int) -> torch.Tensor:
    """A fixed split as int64 [rows, 2049] (utils/prepare_data.py:40-48): the file must hold exactly that tensor and
    its pinned hash; anything else raises ValueError (a file name without a pinned hash raises KeyError, as there)."""
    data = torch.load(path, map_location='cpu', weights_only=True)
    if not isinstance(data, torch.Tensor) or tuple(data.shape) != (rows, SEQ):
        raise ValueError(f'{path}: expected a [{rows}, {SEQ}] token tensor')
    expected = EXPECTED[Path(path).name]
    if expected is not None and token_hash(data) != expected:
        raise ValueError(f'{path}: token hash mismatch; rerun utils/prepare_data.py')
    return data.long()


def load_model(state_dict, device, model_file=None, config=None):
    """The fixed architecture with these weights (utils/eval.py:38-45); a missing, extra or reshaped tensor is an
    error. `config` (a GPTConfig) defaults to the fixed model's."""
    from .model import GPT, GPTConfig
    if model_file is not None:
        raise ValueError('noise_amd evaluates the fixed model only; a track 3 model file is another architecture')
    with torch.device('meta'):
        model = GPT(config if config is not None else GPTConfig())
    model.to_empty(device=device)
    model.init_weights()  # rotary tables, and the bfloat16 storage of the embeddings
    model.load_state_dict(state_dict, strict=True)
    return model.eval().requires_grad_(False)


@torch.no_grad()
def evaluate(state_dict, data_dir='data', batch_size=16, model_file=None, *, rows=None, config=None):
    """Mean loss over all validation predictions (utils/eval.py:48-66). Under torch.distributed the rows are split
    across ranks and the sums all-reduced. `rows` (int64 [n, T + 1]) replaces the validation file when given."""
    rank, world = (dist.get_rank(), dist.get_world_size()) if dist.is_initialized() else (0, 1)
    device = torch.device('cuda', torch.cuda.current_device())
    model = load_model(state_dict, device, model_file, config)
    if rows is None:
        rows = load_rows(Path(data_dir) / 'val.pt', VAL_ROWS)
    rows = rows[rank::world]
    total = torch.zeros(2, dtype=torch.float64, device=device)  # summed loss, predictions
    for batch in rows.split(batch_size):
        batch = batch.to(device)
        loss = model(batch[:, :-1].contiguous(), batch[:, 1:].contiguous(), loss_reduction='sum')
        total[0] += loss.double()
        total[1] += batch[:, 1:].numel()
    if world > 1:
        dist.all_reduce(total)
    value = (total[0] / total[1]).item()
    if value != value:
        raise FloatingPointError('Non-finite validation loss')
    return value


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument('checkpoint', type=Path, help='A state dict saved by a training script.')
    parser.add_argument('--data-dir', type=Path, default=Path('data'))
    args = parser.parse_args()
    if 'RANK' in os.environ:
        torch.cuda.set_device(int(os.environ['LOCAL_RANK']))
        dist.init_process_group('nccl')
    else:
        torch.cuda.set_device(0)
    state_dict = torch.load(args.checkpoint, map_location='cpu', weights_only=True)
    value = evaluate(state_dict, args.data_dir)
    if not dist.is_initialized() or dist.get_rank() == 0:
        print(json.dumps(dict(checkpoint=str(args.checkpoint), val_loss=value)), flush=True)
    if dist.is_initialized():
        dist.destroy_process_group()


if __name__ == '__main__':
    main()
