"""noise_lowrank_static, the entry point that allocates nothing (its scratch is a static device array), against
noise_lowrank with a caller's workspace, both through the C ABI: the same kernels on the same inputs, so the sums of
squares (and y) must be bit-identical. Two calls in a row, the second smaller, so the second runs on the first's
leftover scratch contents; sizes past the static array are rejected."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(dev, T, n_in, n_out, m, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(T, n_in, device=dev, generator=g).bfloat16()
    W = (torch.randn(n_out, n_in, device=dev, generator=g) * 0.02).bfloat16()
    rows = torch.randn(m, n_out + n_in + 3, device=dev, generator=g)
    sign = torch.randn(m, device=dev, generator=g) * 1e-2
    return x, W, rows, sign


def _run(lib_call, name, dev, x, mode, W, rows, sign, T, n_in, n_out, m, y=None, ws=None):
    from noise_amd import _lib
    out = torch.full((m,), float('nan'), device=dev)
    args = [_lib.ptr(x), mode, _lib.ptr(W), _lib.ptr(rows), rows.shape[1], 3, 3 + n_out, _lib.ptr(sign), m, T, n_in,
            n_out, _lib.ptr(y), _lib.ptr(out)]
    if ws is not None:
        args += [_lib.ptr(ws), ws.numel()]
    lib_call(name, *args, _lib.stream(dev))
    return out


@pytest.mark.parametrize('order', ['large_then_small'])
def test_static_entry_point_matches_workspace_entry_point(dev, order):
    from noise_amd import _lib
    lib = _lib.lib()
    cases = [(4096, 512, 2048, 64, 1), (1024, 128, 512, 20, 2)]  # (T, in, out, members, x_shared): second smaller
    for T, n_in, n_out, m, mode in cases:
        print(f'noise_lowrank_static T={T} in={n_in} out={n_out} m={m} x_shared={mode}', flush=True)
        x, W, rows, sign = _inputs(dev, T, n_in, n_out, m, seed=T + m)
        need = lib.noise_lowrank_workspace(m, T, n_in, n_out, 1)
        assert need <= 16 << 20
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        want = _run(_lib.call, 'noise_lowrank', dev, x, mode, W, rows, sign, T, n_in, n_out, m, ws=ws)
        got = _run(_lib.call, 'noise_lowrank_static', dev, x, mode, W, rows, sign, T, n_in, n_out, m)
        torch.cuda.synchronize()
        assert torch.isfinite(want).all()
        assert torch.equal(got, want), (got - want).abs().max().item()
    # with y stored (every element formed)
    T, n_in, n_out, m = 512, 64, 256, 5
    print(f'noise_lowrank_static with y T={T} in={n_in} out={n_out} m={m}', flush=True)
    x, W, rows, sign = _inputs(dev, T, n_in, n_out, m, seed=9)
    ws = torch.empty(lib.noise_lowrank_workspace(m, T, n_in, n_out, 1), dtype=torch.uint8, device=dev)
    y_ws, y_st = (torch.empty(m, T, n_out, device=dev) for _ in range(2))
    s_ws = _run(_lib.call, 'noise_lowrank', dev, x, 1, W, rows, sign, T, n_in, n_out, m, y=y_ws, ws=ws)
    s_st = _run(_lib.call, 'noise_lowrank_static', dev, x, 1, W, rows, sign, T, n_in, n_out, m, y=y_st)
    torch.cuda.synchronize()
    assert torch.equal(y_st, y_ws) and torch.equal(s_st, s_ws)


def test_static_entry_point_rejects_sizes_past_its_array(dev):
    from noise_amd import _lib
    T, n_in, n_out, m = 65536, 512, 2048, 128
    assert _lib.lib().noise_lowrank_workspace(m, T, n_in, n_out, 1) > 16 << 20
    x = torch.zeros(T, n_in, dtype=torch.bfloat16, device=dev)
    W = torch.zeros(n_out, n_in, dtype=torch.bfloat16, device=dev)
    rows = torch.zeros(m, n_out + n_in + 3, device=dev)
    sign = torch.zeros(m, device=dev)
    with pytest.raises(ValueError, match='static array'):
        _run(_lib.call, 'noise_lowrank_static', dev, x, 1, W, rows, sign, T, n_in, n_out, m)
    with pytest.raises(ValueError, match='x_shared 1 or 2'):
        _run(_lib.call, 'noise_lowrank_static', dev, x, 0, W, rows, sign, T, n_in, n_out, m)


def _capture_and_check(dev, T, n_in, n_out, m, seed, eager_first):
    """Captures noise_lowrank_static into a HIP graph on torch's capture stream (a side stream), replays it three
    times with eager work and synchronizations between the replays, and holds every replay bit-equal to
    noise_lowrank's result on the same inputs. eager_first: noise_lowrank (and so the kernels' one-time attribute
    set-up) runs before the capture; otherwise the static entry point's first call on the device, with its scratch
    address lookup, is the captured one."""
    from noise_amd import _lib
    lib = _lib.lib()
    x, W, rows, sign = _inputs(dev, T, n_in, n_out, m, seed=seed)
    ws = torch.empty(lib.noise_lowrank_workspace(m, T, n_in, n_out, 1), dtype=torch.uint8, device=dev)
    want = None
    if eager_first:
        want = _run(_lib.call, 'noise_lowrank', dev, x, 1, W, rows, sign, T, n_in, n_out, m, ws=ws)
    torch.cuda.synchronize()
    out = torch.full((m,), float('nan'), device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.call('noise_lowrank_static', _lib.ptr(x), 1, _lib.ptr(W), _lib.ptr(rows), rows.shape[1], 3, 3 + n_out,
                  _lib.ptr(sign), m, T, n_in, n_out, None, _lib.ptr(out), _lib.stream(dev))
    if want is None:
        want = _run(_lib.call, 'noise_lowrank', dev, x, 1, W, rows, sign, T, n_in, n_out, m, ws=ws)
    torch.cuda.synchronize()
    assert torch.isfinite(want).all()
    for rep in range(3):
        out.fill_(float('nan'))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), (rep, (out - want).abs().max().item())
        x2, W2, r2, s2 = _inputs(dev, 1024, 128, 512, 9, seed=rep)  # eager use of the same scratch in between
        _run(_lib.call, 'noise_lowrank_static', dev, x2, 1, W2, r2, s2, 1024, 128, 512, 9)
        torch.cuda.synchronize()


def test_static_entry_point_replays_under_graph_capture(dev):
    print('noise_lowrank_static under graph capture, after eager calls', flush=True)
    _capture_and_check(dev, 4096, 512, 2048, 64, seed=31, eager_first=True)


def test_static_entry_point_first_call_under_graph_capture():
    """The same in a fresh process whose first call of the library on the device is the captured one."""
    import subprocess
    import sys
    from pathlib import Path
    if not torch.cuda.is_available():
        pytest.skip('no GPU')
    root = Path(__file__).resolve().parents[1]
    code = ('import sys, torch; sys.path.insert(0, %r); from tests import test_zz_no_alloc as t; '
            't._capture_and_check(torch.device("cuda", 0), 2048, 512, 1024, 32, seed=37, eager_first=False); '
            'print("ok", flush=True)' % str(root))
    print('noise_lowrank_static first call under graph capture, fresh process', flush=True)
    r = subprocess.run([sys.executable, '-c', code], cwd=str(root), capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith('ok'), (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
