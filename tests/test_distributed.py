"""The world > 1 branches on CPU: two processes over gloo (127.0.0.1) run the rank-dependent host logic of the
population step (each rank's share of the members, the all_gather of the losses), the validation (each rank's rows,
the all-reduced totals) and the trainer's split check, and compare with what one process computes. No GPU call is
made: the losses stand in as a function of each member's (direction, sign, sequence)."""
import os
import socket

import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

WORLD = 2


def _stand_in_losses(direction, sign, seq):
    # distinct per member, so any reordering or duplication of members changes the vector
    return (direction * 16 + seq).to(torch.float32) + 0.25 * sign


def _worker(rank, world, port, pairs, n_seq, chunk):
    os.environ['MASTER_ADDR'] = '127.0.0.1'
    os.environ['MASTER_PORT'] = str(port)
    dist.init_process_group('gloo', rank=rank, world_size=world)
    try:
        from noise_amd.eval import Scorer, _share
        from noise_amd.model import GPT, GPTConfig
        from noise_amd.population import CHUNK, Eggroll
        from noise_amd.train import Trainer

        with torch.device('meta'):
            model = GPT(GPTConfig())

        # population step: this rank's members, then the gathered losses in the one-process member order
        es = Eggroll(model, pairs, rank=rank, world=world, chunk=chunk)
        es.device = torch.device('cpu')
        members, d, s, q = es.member_layout(n_seq)
        assert d.numel() == members // world
        full = es.gather(_stand_in_losses(d, s, q))
        one = Eggroll(model, pairs, rank=0, world=1, chunk=chunk)
        one.device = torch.device('cpu')
        _, d1, s1, q1 = one.member_layout(n_seq)
        assert torch.equal(full, _stand_in_losses(d1, s1, q1))

        # validation: the ranks' rows partition the rows in order, and the all-reduced totals give the global mean
        rows = torch.arange(11 * 5, dtype=torch.int64).reshape(11, 5)
        share = _share(rows)
        shares = [None] * world
        dist.all_gather_object(shares, share.tolist())
        assert sum(shares, []) == rows.tolist()
        scorer = object.__new__(Scorer)
        scorer.totals = torch.tensor([float(share.sum()), float(share.numel())], dtype=torch.float64)
        assert abs(scorer.value() - rows.double().mean().item()) < 1e-12

        # the trainer splits the pairs into whole chunks per rank
        train_rows = torch.zeros(64, 9, dtype=torch.int64)
        assert Trainer(train_rows, pairs=world * CHUNK).config()['world'] == world
        with pytest.raises(ValueError, match='whole chunks'):
            Trainer(train_rows, pairs=3 * CHUNK)
    finally:
        dist.destroy_process_group()


def _free_port():
    with socket.socket() as sk:
        sk.bind(('127.0.0.1', 0))
        return sk.getsockname()[1]


@pytest.mark.parametrize('pairs,n_seq,chunk', [(64, 4, 8), (96, 2, 4)])
def test_two_ranks_reproduce_the_one_process_population_and_validation(pairs, n_seq, chunk):
    mp.spawn(_worker, args=(WORLD, _free_port(), pairs, n_seq, chunk), nprocs=WORLD, join=True)


def test_one_process_trainer_accepts_the_split_two_ranks_reject():
    from noise_amd.population import CHUNK
    from noise_amd.train import Trainer
    assert Trainer(torch.zeros(64, 9, dtype=torch.int64), pairs=3 * CHUNK).config()['world'] == 1
