"""The score path's host logic (noise_amd/eval.py, mirroring utils/eval.py and utils/prepare_data.py:20-48) on the
CPU: the token hash's byte layout, the pinned-file checks of load_rows and the strict weight loading."""
import hashlib

import pytest
import torch

from noise_amd import eval as ne


def test_token_hash_is_sha256_of_int32_little_endian_bytes():
    rows = torch.tensor([[1, 2], [-1, 4096]], dtype=torch.int64)
    raw = (b'\x01\x00\x00\x00' b'\x02\x00\x00\x00' b'\xff\xff\xff\xff' b'\x00\x10\x00\x00')
    assert ne.token_hash(rows) == hashlib.sha256(raw).hexdigest()
    assert ne.token_hash(rows.to(torch.int32)) == ne.token_hash(rows)  # independent of the stored dtype


def test_pinned_hashes_and_shapes_are_the_references():
    assert (ne.SEQ, ne.TRAIN_ROWS, ne.VAL_ROWS) == (2049, 14648, 544)
    assert ne.VAL_ROWS * (ne.SEQ - 1) == 1_114_112 and ne.TRAIN_ROWS * (ne.SEQ - 1) == 29_999_104
    assert set(ne.EXPECTED) == {'train.pt', 'val.pt'} and all(len(h) == 64 for h in ne.EXPECTED.values())


def _rows(n, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 4096, (n, ne.SEQ), generator=g, dtype=torch.int32)


def test_load_rows_checks_shape_hash_and_name(tmp_path, monkeypatch):
    rows = _rows(ne.VAL_ROWS)
    path = tmp_path / 'val.pt'
    torch.save(rows, path)
    with pytest.raises(ValueError, match='hash mismatch'):  # synthetic rows are not the pinned data
        ne.load_rows(path, ne.VAL_ROWS)
    with pytest.raises(ValueError, match='token tensor'):
        ne.load_rows(path, ne.VAL_ROWS - 1)
    torch.save({'rows': rows}, tmp_path / 'dict.pt')
    with pytest.raises(ValueError, match='token tensor'):
        ne.load_rows(tmp_path / 'dict.pt', ne.VAL_ROWS)
    torch.save(rows, tmp_path / 'other.pt')
    with pytest.raises(KeyError):  # a split without a pinned hash
        ne.load_rows(tmp_path / 'other.pt', ne.VAL_ROWS)
    monkeypatch.setitem(ne.EXPECTED, 'val.pt', ne.token_hash(rows))
    got = ne.load_rows(path, ne.VAL_ROWS)
    assert got.dtype == torch.int64 and torch.equal(got, rows.long())


def test_load_model_is_strict(tmp_path):
    from noise_amd.model import GPTConfig
    cfg = GPTConfig(sequence_len=256)
    ref = ne.load_model(_state(cfg), 'cpu', config=cfg)
    sd = ref.state_dict()
    assert list(sd) == list(_state(cfg))
    missing = dict(sd)
    missing.pop('lm_head.weight')
    with pytest.raises(RuntimeError):
        ne.load_model(missing, 'cpu', config=cfg)
    extra = dict(sd, bogus=torch.zeros(1))
    with pytest.raises(RuntimeError):
        ne.load_model(extra, 'cpu', config=cfg)
    with pytest.raises(ValueError):
        ne.load_model(sd, 'cpu', model_file='train/arch/model.py', config=cfg)


def _state(cfg):
    from noise_amd.model import GPT
    torch.manual_seed(0)
    m = GPT(cfg)
    m.init_weights()
    return m.state_dict()


def test_head_error_takes_device_tensors_only():
    from noise_amd import dust
    raw = torch.zeros(1, 4, 256)
    with pytest.raises(ValueError):
        dust.head_error(raw, torch.zeros(1, 4, dtype=torch.long), torch.zeros(1, 4), draws=16)
    assert dust.chunk_size(48, 16) == 16 and dust.chunk_size(24, 16) == 12 and dust.chunk_size(7, 16) == 7


def test_training_run_checks_its_arguments_first(tmp_path):
    """Pairs that do not split into whole chunks, too few rows for one update, or a used output directory fail before
    any GPU work."""
    import torch
    from noise_amd.train import train
    rows = torch.zeros(16, 2049, dtype=torch.int64)
    with pytest.raises(ValueError, match='whole chunks'):
        train(output=tmp_path / 'o', pairs=100, rows=rows)
    with pytest.raises(ValueError, match='no update'):
        train(output=tmp_path / 'o', pairs=256, rows=rows[:7])
