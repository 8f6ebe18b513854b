"""EGGROLL's population training step on the MI355X kernels, with the reference's host API
(archive/10M/train/val/eggroll.py): lowrank, lowrank_embed, population_loss and Eggroll(model, pairs, rank, world)
with offsets(step), noise(offsets, directions) and step(x, y, optimizer, step).

A direction's noise is a set of contiguous slices of one virtual N(0,1) buffer of 2^28 values at per-step offsets
(eggroll.py:107-128); here the buffer is a counter-based generator (Philox4x32-10 + Box-Muller) evaluated on the GPU,
so nothing of 1 GiB is ever stored. All of a direction's slices sit side by side in one noise row, in
named_parameters() order; the forward kernels read a member's a and b vectors from its row.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib

NOISE = 2 ** 28
SEED = 0
SIGMA = 0.002
CHUNK = 256


class NoiseLayout:
    """Columns of every parameter's (a | b) slice (eps for 1-D parameters) in a noise row."""

    def __init__(self, model):
        self.names, self.shapes, self.widths, self.col0 = [], [], [], []
        col = 0
        for name, p in model.named_parameters():
            w = int(sum(p.shape))
            self.names.append(name)
            self.shapes.append(tuple(p.shape))
            self.widths.append(w)
            self.col0.append(col)
            col += w
        self.stride = col
        self.index = {n: i for i, n in enumerate(self.names)}
        self._widths_c = None

    @property
    def widths_c(self):
        """The widths as a ctypes int64 array (built on first use: the constructor stays plain Python, which
        torch.compile traces without a graph break)."""
        if self._widths_c is None:
            self._widths_c = (ctypes.c_int64 * len(self.widths))(*self.widths)
        return self._widths_c

    def col(self, name):
        return self.col0[self.index[name]]

    def cols(self, n_layer):
        """The slice columns the population forward reads, as a flat list: resid_lambdas, x0_lambdas, wte, lm_head,
        then per block c_q, c_k, c_v, c_proj, ve_gate, c_fc, mlp_proj, ve (-1 on blocks without value embeddings)."""
        out = [self.col('resid_lambdas'), self.col('x0_lambdas'), self.col('transformer.wte.weight'),
               self.col('lm_head.weight')]
        for i in range(n_layer):
            pre = f'transformer.h.{i}.'
            ve = pre + 'attn.ve_gate.weight' in self.index
            out += [self.col(pre + 'attn.c_q.weight'), self.col(pre + 'attn.c_k.weight'),
                    self.col(pre + 'attn.c_v.weight'), self.col(pre + 'attn.c_proj.weight'),
                    self.col(pre + 'attn.ve_gate.weight') if ve else -1, self.col(pre + 'mlp.c_fc.weight'),
                    self.col(pre + 'mlp.c_proj.weight'), self.col(f'value_embeds.{i}.weight') if ve else -1]
        return out

    def struct(self, rows, n_layer):
        return perturbation_struct(rows, self.stride, self.cols(n_layer), n_layer)


def perturbation_struct(rows, stride, cols, n_layer):
    """The noise_perturbation struct: rows fp32 [n_rows, stride] (or None) and the flat column list of
    NoiseLayout.cols."""
    s = _lib.NoisePerturbation()
    s.rows = None if rows is None else rows.data_ptr()
    s.stride = stride
    s.n_rows = 0 if rows is None else rows.shape[0]
    s.resid_lambdas, s.x0_lambdas, s.wte, s.lm_head = cols[:4]
    for i in range(n_layer):
        c = cols[4 + 8 * i: 12 + 8 * i]
        s.c_q[i], s.c_k[i], s.c_v[i], s.c_proj[i], s.c_fc[i], s.mlp_proj[i] = c[0], c[1], c[2], c[3], c[5], c[6]
        if c[4] >= 0:
            s.ve_gate[i], s.ve[i] = c[4], c[7]
    return s


_WORKSPACE = {}


def workspace(device, nbytes):
    """One cached device workspace per device, grown on demand (the kernels themselves never allocate)."""
    buf = _WORKSPACE.get(device)
    if buf is None or buf.numel() < nbytes:
        _WORKSPACE.pop(device, None)
        buf = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        _WORKSPACE[device] = buf
    return buf


def _check_tables(tokens, targets, member_seq, noise, member_row, member_sign, layout, dev, values):
    """The member tables and token rows as the kernels read them: device, dtype, contiguity and sizes always; with
    values, also every member_seq in [0, n_seq) and member_row in [0, n_rows) (a device-to-host sync). The kernels
    guard the same ranges themselves (an out-of-range member's loss is NaN), so callers that build the tables
    themselves skip the sync."""
    if tokens.dim() != 2 or tokens.dtype != torch.int64 or not tokens.is_contiguous():
        raise ValueError(f'tokens must be contiguous int64 [n_seq, T], got {tokens.dtype} {tuple(tokens.shape)}')
    if targets is not None and (targets.shape != tokens.shape or targets.dtype != torch.int64
                                or not targets.is_contiguous()):
        raise ValueError('targets must be contiguous int64 of the tokens\' shape')
    members = member_seq.numel()
    tables = [('member_seq', member_seq, torch.int32)]
    if noise is not None:
        if noise.dim() != 2 or noise.dtype != torch.float32 or not noise.is_contiguous() or \
                noise.shape[1] != layout.stride:
            raise ValueError(f'noise must be contiguous fp32 [n_rows, {layout.stride}], got {noise.dtype} '
                             f'{tuple(noise.shape)}')
        tables += [('member_row', member_row, torch.int32), ('member_sign', member_sign, torch.float32)]
    for name, t, dt in tables:
        if t is None or t.dtype != dt or t.dim() != 1 or t.numel() != members or not t.is_contiguous():
            raise ValueError(f'{name} must be contiguous {dt} [{members}]')
    for name, t in [('tokens', tokens), ('targets', targets), ('noise', noise)] + [(n, t) for n, t, _ in tables]:
        if t is not None and t.device != dev:
            raise ValueError(f'{name} is on {t.device}, the model on {dev}')
    if values:
        checks = [('member_seq', member_seq, tokens.shape[0])]
        if noise is not None:
            checks.append(('member_row', member_row, noise.shape[0]))
        for name, t, n in checks:
            lo, hi = int(t.min()), int(t.max())
            if lo < 0 or hi >= n:
                raise ValueError(f'{name} holds entries in [{lo}, {hi}], outside [0, {n})')


def run_forward(model, tokens, targets, member_seq, noise=None, member_row=None, member_sign=None, layout=None,
                want_logits=False, want_tokens=False, want_sum=True, check_tables=True):
    """One call of noise_population_forward: members evaluate rows of tokens [n_seq, T] (T % 128 == 0).

    noise: fp32 rows [n_rows, layout.stride] or None; member_row / member_sign: int32 / fp32 [members].
    check_tables: also check the table entries' ranges on the host (a sync); callers that build their own tables
    pass False (the kernels still turn an out-of-range member into a NaN loss)."""
    s, keep, dev = model.packed()
    n_seq, T = tokens.shape
    members = member_seq.numel()
    cos, sin = model.rope_tables(T)
    s.rope_cos, s.rope_sin = cos.data_ptr(), sin.data_ptr()
    layout = layout or NoiseLayout(model)
    if noise is None:
        member_row = torch.zeros(members, dtype=torch.int32, device=dev)
        member_sign = torch.zeros(members, dtype=torch.float32, device=dev)
    _check_tables(tokens, targets, member_seq, noise, member_row, member_sign, layout, dev, check_tables)
    pert = layout.struct(noise, model.config.n_layer)
    out = {}
    out['loss_sum'] = torch.empty(members, dtype=torch.float32, device=dev) if (targets is not None and want_sum) else None
    out['token_loss'] = torch.empty(members * T, dtype=torch.float32, device=dev) if want_tokens else None
    out['logits'] = (torch.empty(members * T, model.config.vocab_size, dtype=torch.float32, device=dev)
                     if want_logits else None)
    nbytes = _lib.lib().noise_population_forward_workspace(members, T)
    ws = workspace(dev, nbytes)
    _lib.call('noise_population_forward', ctypes.byref(s), ctypes.byref(pert), _lib.ptr(tokens), _lib.ptr(targets),
              n_seq, T, _lib.ptr(member_seq), _lib.ptr(member_row), _lib.ptr(member_sign), members,
              _lib.ptr(out['loss_sum']), _lib.ptr(out['token_loss']), _lib.ptr(out['logits']), _lib.ptr(ws),
              ws.numel(), _lib.stream(dev))
    return out


def _lowrank(x, weight, a, b, sign):
    """x [m, T, in] (or one [T, in] shared by every member, which the reference's broadcasting also takes) through
    W [out, in] + sign a b^T, one (a [m, out], b [m, in], sign [m]) per member (eggroll.py:56-58): fp32 [m, T, out].
    Per-member x: one grouped bf16 MFMA GEMM with the rank-1 term in its epilogue. Shared x: x W^T once per tile,
    every member's rank-1 term added to that tile."""
    _lib.require_device(x, weight, a, b, sign)
    if x.dim() not in (2, 3) or weight.dim() != 2 or x.shape[-1] != weight.shape[1]:
        raise ValueError(f'lowrank: x {tuple(x.shape)} and weight {tuple(weight.shape)} do not match')
    m = sign.numel()
    T, n_in = x.shape[-2], x.shape[-1]
    n_out = weight.shape[0]
    if a.shape != (m, n_out) or b.shape != (m, n_in) or (x.dim() == 3 and x.shape[0] != m):
        raise ValueError('lowrank: a [m, out], b [m, in] and sign [m] must match x and weight')
    shared = x.dim() == 2
    xb = x.to(torch.bfloat16).contiguous()
    wb = weight.to(torch.bfloat16).contiguous()
    rows = torch.cat([a.float(), b.float()], 1).contiguous()
    sg = sign.float().contiguous()
    y = torch.empty(m, T, n_out, dtype=torch.float32, device=x.device)
    ws = workspace(x.device, _lib.lib().noise_lowrank_workspace(m, T, n_in, n_out, int(shared)))
    _lib.call('noise_lowrank', _lib.ptr(xb), int(shared), _lib.ptr(wb), _lib.ptr(rows), rows.shape[1], 0, n_out,
              _lib.ptr(sg), m, T, n_in, n_out, _lib.ptr(y), None, _lib.ptr(ws), ws.numel(), _lib.stream(x.device))
    return y


LOWRANK_MODES = {'expansion': 1, 'direct': 2}


def lowrank_sumsq(x, weight, rows, a_off, b_off, sign, mode='expansion'):
    """Per-member sums of squares S_i = sum_{t,o} y_i[t, o]^2 of y_i = x W^T + sign_i (x . b_i) a_i^T with x [T, in]
    shared by every member (config 2's single perturbed linear), y never stored; a_i / b_i are columns
    a_off .. a_off + out and b_off .. b_off + in of fp32 noise row i [m, stride]. mode 'expansion': the per-member
    terms of the expanded square on the MFMA units; 'direct': every y element formed and squared. fp32 [m]."""
    _lib.require_device(x, weight, rows, sign)
    if mode not in LOWRANK_MODES:
        raise ValueError(f'lowrank_sumsq: mode must be one of {sorted(LOWRANK_MODES)}')
    if x.dim() != 2 or weight.dim() != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError(f'lowrank_sumsq: x [T, in] {tuple(x.shape)} and weight [out, in] {tuple(weight.shape)}')
    m = sign.numel()
    T, n_in = x.shape
    n_out = weight.shape[0]
    if rows.dim() != 2 or rows.shape[0] < m or a_off < 0 or b_off < 0 or a_off + n_out > rows.shape[1] \
            or b_off + n_in > rows.shape[1]:
        raise ValueError('lowrank_sumsq: the a / b slices do not fit the noise rows')
    xb = x.to(torch.bfloat16).contiguous()
    wb = weight.to(torch.bfloat16).contiguous()
    rf = rows.float().contiguous()
    sg = sign.float().contiguous().view(-1)
    out = torch.empty(m, dtype=torch.float32, device=x.device)
    ws = workspace(x.device, _lib.lib().noise_lowrank_workspace(m, T, n_in, n_out, 1))
    _lib.call('noise_lowrank', _lib.ptr(xb), LOWRANK_MODES[mode], _lib.ptr(wb), _lib.ptr(rf), rf.shape[1], a_off,
              b_off, _lib.ptr(sg), m, T, n_in, n_out, None, _lib.ptr(out), _lib.ptr(ws), ws.numel(),
              _lib.stream(x.device))
    return out


def _lowrank_embed(weight, a, b, idx, sign):
    """Embedding rows of W [V, d] + sign a b^T for token ids idx [T] (eggroll.py:61-63): fp32 [m, T, d] on
    noise_lowrank_embed, from a [m, V], b [m, d], sign [m] (W fp32 or bf16)."""
    _lib.require_device(weight, a, b, idx, sign)
    V, d = weight.shape
    m = a.shape[0]
    if a.shape != (m, V) or b.shape != (m, d) or sign.shape != (m,) or idx.dim() != 1:
        raise ValueError(f'lowrank_embed: W {tuple(weight.shape)}, a {tuple(a.shape)}, b {tuple(b.shape)}, '
                         f'idx {tuple(idx.shape)}, sign {tuple(sign.shape)}')
    w = weight.detach()
    w = w.contiguous() if w.dtype == torch.bfloat16 else w.float().contiguous()
    a32, b32 = a.detach().float().contiguous(), b.detach().float().contiguous()
    ids, s32 = idx.to(torch.int64).contiguous(), sign.detach().float().contiguous()
    out = torch.empty(m, ids.numel(), d, dtype=torch.float32, device=weight.device)
    _lib.call('noise_lowrank_embed', _lib.ptr(w), int(w.dtype == torch.bfloat16), V, d, _lib.ptr(a32), V,
              _lib.ptr(b32), d, _lib.ptr(ids), _lib.ptr(s32), m, ids.numel(), _lib.ptr(out), _lib.stream(weight.device))
    return out


def pack_noise(layout, noise, m, device):
    """name -> (a, b) / eps per-member tensors (the reference's noise dict) -> one fp32 row per member."""
    parts = []
    for name, shape in zip(layout.names, layout.shapes):
        v = noise[name]
        parts.append(torch.cat([v[0], v[1]], 1) if isinstance(v, tuple) else v)
    return torch.cat([p.to(device=device, dtype=torch.float32) for p in parts], 1).contiguous()


def kernel_weights(model, params, T):
    """The device tensors noise_population_forward reads, in the population_forward op's order: resid_lambdas,
    x0_lambdas and wte (fp32), lm_head (bf16), the rotary cos and sin (fp32 [T, 32]), then per block the stacked
    c_q|c_k|c_v, attn.c_proj, mlp.c_fc and mlp.c_proj weights (bf16) and, on blocks with value embeddings, ve_gate and
    the value table (fp32). Plain torch ops on params (name -> tensor), so a compiled caller traces them."""
    bf = lambda t: t.detach().to(torch.bfloat16).contiguous()
    f32 = lambda t: t.detach().to(torch.float32).contiguous()
    cos, sin = model.rope_tables(T)
    out = [f32(params['resid_lambdas']), f32(params['x0_lambdas']), f32(params['transformer.wte.weight']),
           bf(params['lm_head.weight']), cos, sin]
    for i in range(model.config.n_layer):
        pre = f'transformer.h.{i}.'
        out += [bf(torch.cat([params[pre + 'attn.c_q.weight'], params[pre + 'attn.c_k.weight'],
                              params[pre + 'attn.c_v.weight']])),
                bf(params[pre + 'attn.c_proj.weight']), bf(params[pre + 'mlp.c_fc.weight']),
                bf(params[pre + 'mlp.c_proj.weight'])]
        if pre + 'attn.ve_gate.weight' in params:
            out += [f32(params[pre + 'attn.ve_gate.weight']), f32(params[f'value_embeds.{i}.weight'])]
    return out


@torch.library.custom_op('noise_amd::population_forward', mutates_args=())
def population_forward_op(weights: list[torch.Tensor], rows: torch.Tensor, tokens: torch.Tensor,
                          targets: torch.Tensor, member_seq: torch.Tensor, member_row: torch.Tensor,
                          member_sign: torch.Tensor, n_layer: int, vocab: int, windows: list[int],
                          ve_layers: list[int], cols: list[int]) -> torch.Tensor:
    """Per-member summed CE [members] of noise_population_forward: weights as kernel_weights lists them, noise rows
    fp32 [n_rows, stride], tokens / targets int64 [n_seq, T], the member tables int32 / int32 / fp32 [members],
    cols as NoiseLayout.cols. The eager body of the op: it builds the ctypes structs from the tensors' pointers."""
    dev = tokens.device
    _lib.require_device(rows, tokens, targets, member_seq, member_row, member_sign, *weights)
    if len(windows) != n_layer or len(ve_layers) != n_layer or len(cols) != 4 + 8 * n_layer or \
            len(weights) != 6 + 4 * n_layer + 2 * sum(1 for v in ve_layers if v):
        raise ValueError('population_forward: weights, windows, ve_layers and cols do not match n_layer')
    if n_layer > _lib.MAX_LAYERS:
        raise ValueError(f'n_layer {n_layer} > {_lib.MAX_LAYERS}')
    n_seq, T = tokens.shape
    members = member_seq.numel()
    s = _lib.NoiseGpt()
    s.n_layer, s.vocab, s.padded_vocab = n_layer, vocab, weights[3].shape[0]
    s.resid_lambdas, s.x0_lambdas, s.wte, s.lm_head, s.rope_cos, s.rope_sin = (w.data_ptr() for w in weights[:6])
    k = 6
    for i in range(n_layer):
        L = s.layers[i]
        L.w_qkv, L.w_proj, L.w_fc, L.w_mlp_proj = (w.data_ptr() for w in weights[k:k + 4])
        k += 4
        if ve_layers[i]:
            L.w_gate, L.ve = weights[k].data_ptr(), weights[k + 1].data_ptr()
            k += 2
        L.window = int(windows[i])

    class _Layout:  # the stride the table checks compare against
        stride = rows.shape[1]
    _check_tables(tokens, targets, member_seq, rows, member_row, member_sign, _Layout, dev, False)
    pert = perturbation_struct(rows, rows.shape[1], cols, n_layer)
    loss = torch.empty(members, dtype=torch.float32, device=dev)
    ws = workspace(dev, _lib.lib().noise_population_forward_workspace(members, T))
    _lib.call('noise_population_forward', ctypes.byref(s), ctypes.byref(pert), _lib.ptr(tokens), _lib.ptr(targets),
              n_seq, T, _lib.ptr(member_seq), _lib.ptr(member_row), _lib.ptr(member_sign), members, _lib.ptr(loss),
              None, None, _lib.ptr(ws), ws.numel(), _lib.stream(dev))
    return loss


@population_forward_op.register_fake
def _(weights, rows, tokens, targets, member_seq, member_row, member_sign, n_layer, vocab, windows, ve_layers, cols):
    return member_seq.new_empty(member_seq.shape, dtype=torch.float32)


@torch.library.custom_op('noise_amd::lowrank', mutates_args=())
def lowrank_op(x: torch.Tensor, weight: torch.Tensor, a: torch.Tensor, b: torch.Tensor,
               sign: torch.Tensor) -> torch.Tensor:
    return _lowrank(x, weight, a, b, sign)


@lowrank_op.register_fake
def _(x, weight, a, b, sign):
    return x.new_empty((sign.numel(), x.shape[-2], weight.shape[0]), dtype=torch.float32)


@torch.library.custom_op('noise_amd::lowrank_embed', mutates_args=())
def lowrank_embed_op(weight: torch.Tensor, a: torch.Tensor, b: torch.Tensor, idx: torch.Tensor,
                     sign: torch.Tensor) -> torch.Tensor:
    return _lowrank_embed(weight, a, b, idx, sign)


@lowrank_embed_op.register_fake
def _(weight, a, b, idx, sign):
    return weight.new_empty((a.shape[0], idx.numel(), weight.shape[1]), dtype=torch.float32)


def lowrank(x, weight, a, b, sign):
    """x [m, T, in] (or one [T, in] shared by every member, which the reference's broadcasting also takes) through
    W [out, in] + sign a b^T, one (a [m, out], b [m, in], sign [m]) per member (eggroll.py:56-58): fp32 [m, T, out],
    as the custom op noise_amd::lowrank (so a compiled caller keeps it in its graph)."""
    return torch.ops.noise_amd.lowrank(x, weight, a, b, sign)


def lowrank_embed(weight, a, b, idx, sign):
    """Embedding rows of W [V, d] + sign a b^T for token ids idx [T] (eggroll.py:61-63): fp32 [m, T, d], as the
    custom op noise_amd::lowrank_embed."""
    return torch.ops.noise_amd.lowrank_embed(weight, a, b, idx, sign)


def population_loss(model, p, noise, sign, idx, targets):
    """Mean cross-entropy [m] of m perturbed models on one sequence (eggroll.py:66-103), the model's weights taken
    from p (name -> tensor, the reference's parameters by name; None: the model's own). noise: name -> (a [m, out],
    b [m, in]) or eps [m, L]. The forward itself is the custom op noise_amd::population_forward, and everything around
    it is plain torch, so torch.compile(population_loss) (the reference compiles it, eggroll.py:115) traces the whole
    call into one graph with no break."""
    params = p if p is not None else dict(model.named_parameters())
    dev = model.lm_head.weight.device
    layout = NoiseLayout(model)
    n_layer = model.config.n_layer
    m, T = sign.shape[0], idx.shape[0]
    rows = pack_noise(layout, noise, m, dev)
    Tp = (T + 127) // 128 * 128
    tok = torch.nn.functional.pad(idx.to(torch.int64), (0, Tp - T)).view(1, Tp).contiguous()
    tg = torch.nn.functional.pad(targets.to(torch.int64), (0, Tp - T), value=-1).view(1, Tp).contiguous()
    ve_layers = [int(f'transformer.h.{i}.attn.ve_gate.weight' in layout.index) for i in range(n_layer)]
    loss = torch.ops.noise_amd.population_forward(
        kernel_weights(model, params, Tp), rows, tok, tg, torch.zeros(m, dtype=torch.int32, device=dev),
        torch.arange(m, dtype=torch.int32, device=dev), sign.to(device=dev, dtype=torch.float32).contiguous(),
        n_layer, model.config.vocab_size, [int(w) for w, _ in model.window_sizes], ve_layers, layout.cols(n_layer))
    return loss / T


class Eggroll:
    """Perturbation bookkeeping of eggroll.py:106-168 on the GPU: per-step offsets from a counter-based generator,
    noise rows generated in place, the population forward in chunks of 2 * chunk members, fitness, the outer-product
    gradient assembly and the optimizer step."""

    def __init__(self, model, pairs, rank=0, world=1, sigma=SIGMA, seed=SEED, chunk=CHUNK):
        self.model, self.pairs, self.rank, self.world = model, pairs, rank, world
        self.sigma, self.seed, self.chunk = sigma, seed, chunk
        self.device = next(model.parameters()).device
        self.params = dict(model.named_parameters())
        self.layout = NoiseLayout(model)
        self.last = {}

    def offsets(self, step):
        """name -> int64 [pairs] offsets for this step (eggroll.py:117-120)."""
        table = self.offset_table(step)
        return {name: table[i] for i, name in enumerate(self.layout.names)}

    def offset_table(self, step):
        out = torch.empty(len(self.layout.names), self.pairs, dtype=torch.int64, device=self.device)
        _lib.call('noise_rng_offsets', self.seed, step, self.layout.widths_c, len(self.layout.names), self.pairs,
                  _lib.ptr(out), _lib.stream(self.device))
        return out

    def rows(self, table, directions):
        """fp32 noise rows [n, stride] of the given directions."""
        directions = directions.to(device=self.device, dtype=torch.int64).contiguous()
        rows = torch.empty(directions.numel(), self.layout.stride, dtype=torch.float32, device=self.device)
        _lib.call('noise_rng_rows', self.seed, _lib.ptr(table), self.pairs, self.layout.widths_c,
                  len(self.layout.names), _lib.ptr(directions), directions.numel(), _lib.ptr(rows),
                  _lib.stream(self.device))
        return rows

    def noise(self, offsets, directions):
        """name -> (a [n, out], b [n, in]) for matrices and embeddings, eps [n, L] for 1-D (eggroll.py:122-128)."""
        table = torch.stack([offsets[n] for n in self.layout.names]).contiguous()
        rows = self.rows(table, directions)
        out = {}
        for name, shape, c0, w in zip(self.layout.names, self.layout.shapes, self.layout.col0, self.layout.widths):
            sl = rows[:, c0:c0 + w]
            out[name] = (sl[:, :shape[0]], sl[:, shape[0]:]) if len(shape) == 2 else sl
        return out

    def member_layout(self, n_seq):
        members = max(2 * self.pairs, 2 * n_seq)
        per_seq, per_rank = members // n_seq, members // self.world
        if per_rank % (2 * self.chunk):
            raise ValueError('each rank must evaluate whole chunks of pairs')
        g = torch.arange(self.rank * per_rank, (self.rank + 1) * per_rank, device=self.device)
        start = g - g % (2 * self.chunk)
        return members, (g // 2) % self.pairs, torch.where(g % 2 == 0, 1.0, -1.0), start // per_seq

    def gather(self, losses):
        """Every rank's per-member losses in rank order, which is the whole population's member order (rank r
        evaluates the r-th contiguous share of it): one all_gather over the default process group
        (eggroll.py:147-150). On one process, `losses` itself."""
        if self.world == 1:
            return losses
        gathered = [torch.empty_like(losses) for _ in range(self.world)]
        torch.distributed.all_gather(gathered, losses)
        return torch.cat(gathered)

    # pairs per chunk of the update: each chunk's noise rows are generated, consumed and dropped
    UPDATE_PAIRS = 1024

    @torch.no_grad()
    def step(self, x, y, optimizer, step):
        """Evaluate this rank's share of the population, gather the losses, rebuild the update everywhere
        (eggroll.py:130-168). Returns the mean population loss (a host sync).

        No population-wide noise is stored: each chunk of the forward generates the rows of its own directions (the
        2 chunk members of a chunk use `chunk` consecutive directions, each with both signs) from the counter stream
        right before it runs, and the update regenerates the rows of UPDATE_PAIRS directions at a time and adds their
        outer products into the gradients."""
        n_seq, T = x.shape
        if T % 128:
            raise ValueError(f'sequence length {T} must be a multiple of 128')
        members, direction, sgn, seq = self.member_layout(n_seq)
        table = self.offset_table(step)
        tokens, targets = x.to(torch.int64).contiguous(), y.to(torch.int64).contiguous()
        per_rank = direction.numel()
        losses = torch.empty(per_rank, dtype=torch.float32, device=self.device)
        m_chunk = 2 * self.chunk
        for c in range(0, per_rank, m_chunk):
            sl = slice(c, c + m_chunk)
            dirs = direction[sl]
            rows = self.rows(table, dirs[0::2])  # members 2i and 2i + 1 share direction dirs[2i]
            local = torch.arange(dirs.numel(), device=self.device, dtype=torch.int32) // 2
            out = run_forward(self.model, tokens, targets, member_seq=seq[sl].to(torch.int32).contiguous(),
                              noise=rows, member_row=local, member_sign=(sgn[sl] * self.sigma).float().contiguous(),
                              layout=self.layout, check_tables=False)
            losses[sl] = out['loss_sum'] / T
        losses = self.gather(losses)
        n_fit = losses.numel() // 2
        fitness = torch.empty(n_fit, dtype=torch.float32, device=self.device)
        weight = torch.empty(self.pairs, dtype=torch.float32, device=self.device)
        _lib.call('noise_fitness', _lib.ptr(losses), losses.numel(), self.pairs, _lib.ptr(fitness), _lib.ptr(weight),
                  _lib.stream(self.device))
        optimizer.zero_grad(set_to_none=True)
        grads, mats, vecs = {}, [], []
        for name, shape, c0 in zip(self.layout.names, self.layout.shapes, self.layout.col0):
            grads[name] = grad = torch.empty(shape, dtype=torch.float32, device=self.device)
            (mats if len(shape) == 2 else vecs).append((c0, shape, grad))
        arr = lambda vals, t: (t * len(vals))(*vals)
        a_off = arr([c0 for c0, _, _ in mats], ctypes.c_int64)
        b_off = arr([c0 + shape[0] for c0, shape, _ in mats], ctypes.c_int64)
        outs = arr([shape[0] for _, shape, _ in mats], ctypes.c_int64)
        ins = arr([shape[1] for _, shape, _ in mats], ctypes.c_int64)
        ptrs = arr([g.data_ptr() for _, _, g in mats], ctypes.c_void_p)
        stream = _lib.stream(self.device)
        for k0 in range(0, self.pairs, self.UPDATE_PAIRS):
            k1 = min(self.pairs, k0 + self.UPDATE_PAIRS)
            rows = self.rows(table, torch.arange(k0, k1, device=self.device))
            w = weight[k0:k1]
            acc = int(k0 > 0)
            for c0, shape, grad in vecs:
                _lib.call('noise_outer_grad', _lib.ptr(rows), self.layout.stride, c0, -1, _lib.ptr(w), k1 - k0, 1,
                          shape[0], -1.0 / n_fit, acc, _lib.ptr(grad), stream)
            # every matrix's outer-product sum over this chunk of directions in one grouped launch (eggroll.py:155-163)
            _lib.call('noise_outer_grad_batch', _lib.ptr(rows), self.layout.stride, _lib.ptr(w), k1 - k0, len(mats),
                      a_off, b_off, outs, ins, ptrs, -1.0 / n_fit, acc, stream)
        for name in self.layout.names:
            self.params[name].grad = grads[name].to(self.params[name].dtype)
        optimizer.step()
        self.last = dict(losses=losses, fitness=fitness, weight=weight)
        return losses.mean().item()
