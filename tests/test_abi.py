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
    assert lib.noise_abi_version() == 1


def test_argument_errors_raise_before_any_gpu_call():
    from noise_amd import _lib
    w = (ctypes.c_int64 * 1)(10)
    with pytest.raises(ValueError, match='n_params'):
        _lib.call('noise_rng_offsets', 0, 0, w, 0, 4, None, None)
    with pytest.raises(ValueError, match='pairs'):
        _lib.call('noise_rng_offsets', 0, 0, w, 1, 0, None, None)
    with pytest.raises(ValueError, match='multiple of 128'):
        _lib.call('noise_credit_lse', ctypes.c_void_p(16), ctypes.c_void_p(16), 2, 100, 10, ctypes.c_void_p(16), None)
    with pytest.raises(ValueError, match='even'):
        _lib.call('noise_fitness', ctypes.c_void_p(16), 3, 1, ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert _lib.lib().noise_population_forward_workspace(0, 128) == 0
    assert _lib.lib().noise_population_forward_workspace(2, 128) > 2 * 128 * 512 * 8


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
