"""The C-ABI library loads and exports every entry point include/noise_amd.h declares; host-side argument checks turn
into the documented Python exceptions (no GPU call is made); host logic mirrors the reference's layout."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / 'include' / 'noise_amd.h').read_text()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(noise_[a-z0-9_]+)\s*\(', text)))


def test_library_exports_every_declared_symbol():
    from noise_amd import _lib
    lib = _lib.lib()
    declared = _declared()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.EXPORTS)
    assert lib.noise_abi_version() == 5 == _lib.ABI_VERSION


def test_argument_errors_raise_before_any_gpu_call():
    from noise_amd import _lib
    w = (ctypes.c_int64 * 1)(10)
    with pytest.raises(ValueError, match='n_params'):
        _lib.call('noise_rng_offsets', 0, 0, w, 0, 4, None, None)
    with pytest.raises(ValueError, match='pairs'):
        _lib.call('noise_rng_offsets', 0, 0, w, 1, 0, None, None)
    with pytest.raises(ValueError, match='multiple of 128'):
        _lib.call('noise_credit_lse', ctypes.c_void_p(16), ctypes.c_void_p(16), 2, 100, 10, ctypes.c_void_p(16), None)
    with pytest.raises(ValueError, match='multiple of 128'):
        _lib.call('noise_credit_lse_bounded', ctypes.c_void_p(16), ctypes.c_void_p(16), 2, 100, 10, ctypes.c_void_p(16),
                  None)
    with pytest.raises(ValueError, match='NULL'):
        _lib.call('noise_credit_lse_bounded', None, ctypes.c_void_p(16), 2, 128, 10, ctypes.c_void_p(16), None)
    with pytest.raises(ValueError, match='even'):
        _lib.call('noise_fitness', ctypes.c_void_p(16), 3, 1, ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert _lib.lib().noise_population_forward_workspace(0, 128) == 0
    assert _lib.lib().noise_population_forward_workspace(2, 128) > 2 * 128 * 512 * 8


def test_credit_operands_must_match_q():
    """A smaller k, lse or hub would be read past its end on the device: every operand's shape is checked first."""
    from noise_amd import credit
    q = torch.zeros(2, 128, 64)
    with pytest.raises(ValueError, match='k '):
        credit.credit_lse(q, torch.zeros(2, 64, 64), 10)
    with pytest.raises(ValueError, match='lse'):
        credit.raw_value_credits(q, q, torch.zeros(2, 64), q, 10)
    with pytest.raises(ValueError, match='hub'):
        credit.raw_value_credits(q, q, torch.zeros(2, 128), torch.zeros(1, 128, 64), 10)
    with pytest.raises(ValueError, match='values'):
        credit.key_context(q, q, torch.zeros(2, 128, 32), q, 10)


def test_member_tables_are_checked_on_the_host():
    """run_forward's host checks (noise_amd.population._check_tables): dtype, shape, contiguity and device always;
    with values, entry ranges: member_seq in [0, n_seq) and member_row in [0, n_rows). The kernels guard the same
    ranges on the device (an out-of-range member's loss is NaN), which the GPU tests cover."""
    from noise_amd.population import _check_tables

    class Lay:
        stride = 10
    cpu = torch.device('cpu')
    tok = torch.zeros(2, 128, dtype=torch.int64)
    rows = torch.zeros(3, 10)
    seq = torch.tensor([0, 1, 0, 1], dtype=torch.int32)
    row = torch.tensor([0, 0, 2, 2], dtype=torch.int32)
    sign = torch.zeros(4)
    _check_tables(tok, tok, seq, rows, row, sign, Lay, cpu, True)
    _check_tables(tok, None, seq, None, None, None, Lay, cpu, True)
    cases = [
        (dict(seq=torch.tensor([0, 1, 2, 1], dtype=torch.int32)), 'member_seq holds'),
        (dict(seq=torch.tensor([0, -1, 0, 1], dtype=torch.int32)), 'member_seq holds'),
        (dict(row=torch.tensor([0, 0, 3, 2], dtype=torch.int32)), 'member_row holds'),
        (dict(row=torch.tensor([0, 0, 2], dtype=torch.int32)), 'member_row must be'),
        (dict(row=row.long()), 'member_row must be'),
        (dict(sign=torch.zeros(4, dtype=torch.float64)), 'member_sign must be'),
        (dict(seq=seq.long()), 'member_seq must be'),
        (dict(rows=torch.zeros(3, 9)), 'noise must be'),
        (dict(tok=tok.int()), 'tokens must be'),
        (dict(tg=tok[:, :64]), 'targets must be'),
    ]
    for change, msg in cases:
        a = dict(tok=tok, tg=tok, seq=seq, rows=rows, row=row, sign=sign)
        a.update(change)
        with pytest.raises(ValueError, match=msg):
            _check_tables(a['tok'], a['tg'], a['seq'], a['rows'], a['row'], a['sign'], Lay, cpu, True)
    # ranges are only checked with values (the kernels guard them on the device)
    _check_tables(tok, tok, torch.tensor([0, 1, 5, 1], dtype=torch.int32), rows, row, sign, Lay, cpu, False)
    with pytest.raises(ValueError, match='the model on meta'):
        _check_tables(tok, tok, seq, rows, row, sign, Lay, torch.device('meta'), False)


def test_compute_on_cpu_tensors_is_refused():
    from noise_amd import credit
    q = torch.zeros(1, 128, 64)
    with pytest.raises(ValueError, match='device'):
        credit.credit_lse(q, q, 10)


def test_noise_layout_matches_param_specs():
    from noise_amd.model import GPT, GPTConfig
    from noise_amd.population import NoiseLayout
    from oracle.model import Config, param_specs
    with torch.device('meta'):
        model = GPT(GPTConfig())
    lay = NoiseLayout(model)
    specs = param_specs(Config())
    assert lay.names == [n for n, _ in specs]
    assert lay.widths == [int(sum(s)) for _, s in specs]
    assert lay.stride == 101_552
    s = lay.struct(None, 8)
    assert s.c_q[0] == lay.col('transformer.h.0.attn.c_q.weight')
    assert s.ve[7] == lay.col('value_embeds.7.weight') and s.ve[0] == 0


def test_state_dict_keys_match_reference_order():
    import json
    from noise_amd.model import GPT, GPTConfig
    with torch.device('meta'):
        model = GPT(GPTConfig())
    order = json.loads((ROOT / 'tests' / 'golden' / 'param_order.json').read_text())
    assert [[n, list(p.shape)] for n, p in model.named_parameters()] == order
    assert list(model.state_dict().keys()) == [n for n, _ in order]


def test_eggroll_member_layout_matches_oracle():
    from noise_amd.model import GPT, GPTConfig
    from noise_amd.population import Eggroll
    from oracle.eggroll import member_layout
    with torch.device('meta'):
        model = GPT(GPTConfig())
    es = Eggroll(model, 12288, chunk=256)
    es.device = torch.device('cpu')
    members, d, s, q = es.member_layout(8)
    rd, rs, rq = member_layout(12288, 8)
    assert members == 24576
    assert np.array_equal(d.numpy(), rd) and np.array_equal(s.numpy(), rs) and np.array_equal(q.numpy(), rq)


def test_dust_and_head_error_arguments_are_checked_before_any_gpu_call():
    from noise_amd import _lib
    p = ctypes.c_void_p(16)
    # head-slab estimator (dust.py:261-303): vocabulary in 256-column slabs, chunks covering the slabs evenly
    with pytest.raises(ValueError, match='multiple of 256'):
        _lib.call('noise_head_error', p, 300, p, p, 1, 4, 300, 16, 16, 0.1, 0, p, p, 1 << 30, None)
    with pytest.raises(ValueError, match='slabs evenly'):
        _lib.call('noise_head_error', p, 512, p, p, 1, 4, 512, 16, 16, 0.1, 0, p, p, 1 << 30, None)
    with pytest.raises(ValueError, match='65,535'):
        _lib.call('noise_head_error', p, 256, p, p, 1, 4, 256, 70000, 16, 0.1, 0, p, p, 1 << 40, None)
    with pytest.raises(ValueError, match='workspace'):
        _lib.call('noise_head_error', p, 256, p, p, 1, 4, 256, 16, 16, 0.1, 0, p, p, 8, None)
    assert _lib.lib().noise_head_error_workspace(8, 512, 16) >= 16 * 8 * 4
    # direct draws' error sums (dust.py:235-259)
    with pytest.raises(ValueError, match='sigma'):
        _lib.call('noise_dust_errors', p, p, 4, 2, 128, 0.0, 0.0, 0, 0, 3, 2048, p, p, 1 << 30, None)
    with pytest.raises(ValueError, match='gamma'):
        _lib.call('noise_dust_errors', p, p, 4, 2, 128, 1.0, 0.4, 0, 0, 3, 2048, p, p, 1 << 30, None)
    with pytest.raises(ValueError, match='site'):
        _lib.call('noise_dust_errors', p, p, 4, 2, 128, 0.0, 0.4, 0, 0, 5, 512, p, p, 1 << 30, None)
    with pytest.raises(ValueError, match='workspace'):
        _lib.call('noise_dust_errors', p, p, 4, 2, 128, 0.0, 0.4, 0, 0, 3, 2048, p, p, 8, None)
    assert _lib.lib().noise_dust_errors_workspace(4, 2, 128) >= 2 * 4 * 2 * 128 * 4
    assert _lib.lib().noise_dust_workspace(0, 2, 128) == 0
    # reruns (dust.py:210-233): the entry, its sites and its captured input
    model = _lib.NoiseGpt()
    model.n_layer = 8
    d = _lib.NoiseDustDraws()
    d.entry, d.sites, d.sigma, d.n_draws = 8, 2, 0.4, 4
    with pytest.raises(ValueError, match='entry'):
        _lib.call('noise_dust_rerun', ctypes.byref(model), ctypes.byref(d), p, p, 2, 128, p, p, 1 << 30, None)
    d.entry, d.sites = 3, 1  # the embedding's site on a block
    with pytest.raises(ValueError, match='do not belong'):
        _lib.call('noise_dust_rerun', ctypes.byref(model), ctypes.byref(d), p, p, 2, 128, p, p, 1 << 30, None)
    d.sites = 4  # a block site without the captured input
    with pytest.raises(ValueError, match='captured input'):
        _lib.call('noise_dust_rerun', ctypes.byref(model), ctypes.byref(d), p, p, 2, 128, p, p, 1 << 30, None)


def test_outer_grad_batch_arguments_are_checked_before_any_gpu_call():
    """Every matrix is validated before the grouped launch: a slice past the noise row, a NULL gradient or a bad
    shape anywhere in the list fails the call."""
    import ctypes
    from noise_amd import _lib
    lib = _lib.lib()
    arr = lambda vals, t: (t * len(vals))(*vals)
    fake = ctypes.c_void_p(256)  # never dereferenced: the checks fail first

    def call(a_off, b_off, out, n_in, grads, stride=100):
        return lib.noise_outer_grad_batch(fake, stride, fake, 10, len(out), arr(a_off, ctypes.c_int64),
                                          arr(b_off, ctypes.c_int64), arr(out, ctypes.c_int64), arr(n_in, ctypes.c_int64),
                                          arr(grads, ctypes.c_void_p), 1.0, 0, None)
    assert call([0, 0], [10, 10], [10, 10], [10, 91], [256, 256]) == 1   # second slice ends past the 100-value row
    assert 'matrix 1: slice beyond the noise row' in lib.noise_last_error().decode()
    assert call([0], [10], [10], [10], [0]) == 1                         # NULL gradient
    assert call([0], [10], [0], [10], [256]) == 1                        # empty matrix
    assert call([-1], [10], [10], [10], [256]) == 1
