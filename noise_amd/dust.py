"""Dust's direct draws (train/val/dust.py:131-259: capture, rerun, direct_errors) and head-slab CE estimator
(:261-303, head_error) on the HIP kernels.

The direct draws rerun the network from a block's captured input with Gaussian jitter at sites of that block, as
DUST.rerun does, on the population forward's kernels: one launch sequence evaluates n draws x the batch's
sequences, the jitter (this library's counter stream, by seed, draw, site and token) added inside the producing
kernel's epilogue; the reward and the error sum (noise_dust_errors) regenerate the same jitter instead of storing it.

DUST.head_error(draws, sigma) reads three things from its DUST instance: the captured lm_head outputs of the clean
forward (self.outputs['lm_head']), the targets (self.y) and the clean per-token losses (self.clean_loss); it draws
its jitter from torch.randn (dust.py:192-193) and batches self.recipe.nrep draws per chunk. `head_error` here takes
those explicitly; the jitter is this library's counter stream, keyed by `seed` (the reference's CUDA generator
stream cannot be reproduced off an NVIDIA GPU), in fp32 where the reference rounds it and the reward-weighted sum
to bf16 (dust.py:281, 299-301).

    error = head_error(raw, y, clean_loss, draws=512, sigma=0.1)   # fp32, raw's shape; 0 past the vocabulary
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

SLAB = 256
# the direct draws' sites inside a block, by block_forward's argument name (dust.py:102-103)
SITES = {'o': 'o@{}', 'attn': 'transformer.h.{}.attn.c_proj', 'fc': 'transformer.h.{}.mlp.c_fc',
         'mlp': 'transformer.h.{}.mlp.c_proj'}
_SITE_ID = {'transformer.wte': 0, 'o': 1, 'attn': 2, 'fc': 3, 'mlp': 4}


def chunk_size(draws: int, cap: int) -> int:
    """The largest count up to cap that divides draws: that many draws share one chunk (dust.py:81-83)."""
    return next(n for n in range(min(cap, draws), 0, -1) if draws % n == 0)


def head_error(raw: torch.Tensor, y: torch.Tensor, clean_loss: torch.Tensor, draws: int, sigma: float = 0.1,
               nrep: int = 16, seed: int = 0, vocab: int | None = None) -> torch.Tensor:
    """Per-token error estimates of the lm_head outputs: raw (b, t, Vp) (cast to bf16, the autocast output the
    reference caches), y int (b, t) with -1 at ignored positions, clean_loss (b, t) the clean forward's per-token CE.
    Each chunk of chunk_size(draws, nrep) draws jitters one 256-column slab of the first `vocab` columns (default: all
    of Vp), in turn; the chunks must cover the slabs evenly, as the reference requires (dust.py:163)."""
    _lib.require_device(raw, y, clean_loss)
    if raw.dim() != 3 or y.shape != raw.shape[:2] or clean_loss.shape != raw.shape[:2]:
        raise ValueError('raw must be (b, t, Vp) with y and clean_loss (b, t)')
    b, t, Vp = raw.shape
    vocab = Vp if vocab is None else int(vocab)
    raw = raw.to(torch.bfloat16).contiguous()
    y = y.to(torch.int64).contiguous()
    clean_loss = clean_loss.float().contiguous()
    error = torch.empty(b, t, Vp, dtype=torch.float32, device=raw.device)
    ws = torch.empty(_lib.lib().noise_head_error_workspace(b * t, vocab, int(draws)), dtype=torch.uint8,
                     device=raw.device)
    _lib.call('noise_head_error', _lib.ptr(raw), Vp, _lib.ptr(y), _lib.ptr(clean_loss), b, t, vocab, int(draws),
              int(nrep), float(sigma), int(seed), _lib.ptr(error), _lib.ptr(ws), ws.numel(), _lib.stream(raw.device))
    return error


def parse_site(model, name):
    """(block or None, site id, width) of a site name: 'transformer.wte', 'o@{i}' or a SITES linear of block i."""
    if name == 'transformer.wte':
        return None, 0, model.config.n_embd
    if name.startswith('o@'):
        return int(name[2:]), 1, model.config.n_embd
    for key, pattern in SITES.items():
        prefix, suffix = pattern.split('{}')
        if key != 'o' and name.startswith(prefix) and name.endswith(suffix):
            i = int(name[len(prefix):len(name) - len(suffix)])
            return i, _SITE_ID[key], 4 * model.config.n_embd if key == 'fc' else model.config.n_embd
    raise ValueError(f'unknown direct-draw site {name!r}')


class Dust:
    """The direct-draw part of DUST (train/val/dust.py:131-259) over the HIP population forward.

    capture(x, y) runs the clean pass, keeping every block's input, the inputs of the writers' linears and the clean
    per-token losses; rerun(n, entry, sites, sigma, draw0) evaluates n jittered draws from block `entry` (None: from
    the token embedding); direct_errors(sites, draws, sigma, entry, gamma) returns the reference's error estimates, and
    reassemble(site, error) turns a site's output error into its weight error (dust.py:386-392). The jitter's draw counter
    advances like the reference's generator, so successive calls use fresh draws; `seed` and `rank` key the stream as
    the reference keys its generator (dust.py:149)."""

    def __init__(self, model, nrep=16, seed=0, rank=0):
        self.model, self.nrep = model, nrep
        self.seed = seed + 3 + 7777 * rank
        self.next_draw = 0

    def capture(self, x, y):
        """The clean pass over tokens x, targets y (b, t): stores every block's (mixed) input and x0, and the clean
        per-token losses (dust.py:195-208); returns the losses (b, t)."""
        from .population import workspace
        model = self.model
        _lib.require_device(x, y)
        b, T = x.shape
        if T % 128:
            raise ValueError(f'sequence length {T} must be a multiple of 128')
        s, keep, dev = model.packed()
        cos, sin = model.rope_tables(T)
        s.rope_cos, s.rope_sin = cos.data_ptr(), sin.data_ptr()
        self._rope = (cos, sin)
        self.x, self.y = x.long().contiguous(), y.long().contiguous()
        self.batch, self.length = b, T
        L, D = model.config.n_layer, model.config.n_embd
        self.blocks = torch.empty(L + 1, b, T, D, dtype=torch.float32, device=dev)
        F = 4 * D
        attn_in = torch.empty(L, b, T, D, dtype=torch.bfloat16, device=dev)
        fc_in = torch.empty(L, b, T, D, dtype=torch.float32, device=dev)
        mlp_in = torch.empty(L, b, T, F, dtype=torch.bfloat16, device=dev)
        loss = torch.empty(b, T, dtype=torch.float32, device=dev)
        ws = workspace(dev, _lib.lib().noise_dust_workspace(1, b, T))
        _lib.call('noise_dust_capture_sites', ctypes.byref(s), _lib.ptr(self.x), _lib.ptr(self.y), b, T, _lib.ptr(loss),
                  _lib.ptr(self.blocks), _lib.ptr(attn_in), _lib.ptr(fc_in), _lib.ptr(mlp_in), _lib.ptr(ws), ws.numel(),
                  _lib.stream(dev))
        # the linears' inputs, by site name, as the reference's hooks keep them (dust.py:173-179)
        self.inputs = {'transformer.wte': self.x}
        for i in range(L):
            self.inputs[SITES['attn'].format(i)] = attn_in[i]
            self.inputs[SITES['fc'].format(i)] = fc_in[i]
            self.inputs[SITES['mlp'].format(i)] = mlp_in[i]
        self.x0 = self.blocks[L]
        self.clean_loss = loss
        return loss

    def rerun(self, n, entry, sites, sigma, draw0):
        """Per-token losses (n, b, t) of draws draw0 .. draw0 + n - 1, each adding sigma a at `sites` (names) of block
        `entry` (None: the token embedding) and rerunning the network from there (dust.py:210-233)."""
        from .population import workspace
        model = self.model
        mask = 0
        for name in sites:
            blk, sid, _ = parse_site(model, name)
            if blk != entry:
                raise ValueError(f'site {name!r} is not in block {entry}')
            mask |= 1 << sid
        s, keep, dev = model.packed()
        cos, sin = self._rope
        s.rope_cos, s.rope_sin = cos.data_ptr(), sin.data_ptr()
        b, T = self.batch, self.length
        d = _lib.NoiseDustDraws()
        d.entry = -1 if entry is None else int(entry)
        if entry is not None:
            d.x_in, d.x0_in = self.blocks[entry].data_ptr(), self.x0.data_ptr()
        d.sites, d.sigma, d.seed, d.draw0, d.n_draws = mask, float(sigma), self.seed, int(draw0), int(n)
        loss = torch.empty(n, b, T, dtype=torch.float32, device=dev)
        ws = workspace(dev, _lib.lib().noise_dust_workspace(n, b, T))
        _lib.call('noise_dust_rerun', ctypes.byref(s), ctypes.byref(d), _lib.ptr(self.x), _lib.ptr(self.y), b, T,
                  _lib.ptr(loss), _lib.ptr(ws), ws.numel(), _lib.stream(dev))
        return loss

    def direct_errors(self, sites, draws, sigma, entry=None, gamma=0.0):
        """One-sided loss drops, centered across each chunk of draws (dust.py:235-259): {site: error (b, t, width)}."""
        from .population import workspace
        n = chunk_size(draws, self.nrep)
        b, T = self.batch, self.length
        dev = self.clean_loss.device
        info = {s: parse_site(self.model, s) for s in sites}
        errors = {s: torch.zeros(b, T, w, dtype=torch.float32, device=dev) for s, (_, _, w) in info.items()}
        for _ in range(draws // n):
            draw0 = self.next_draw
            self.next_draw += n
            loss = self.rerun(n, entry, sites, sigma, draw0)
            ws = workspace(dev, _lib.lib().noise_dust_errors_workspace(n, b, T))  # the rerun's, stream-ordered
            for name, (_, sid, width) in info.items():
                _lib.call('noise_dust_errors', _lib.ptr(loss), _lib.ptr(self.clean_loss), n, b, T, float(gamma),
                          float(sigma), self.seed, draw0, sid, width, _lib.ptr(errors[name]), _lib.ptr(ws),
                          ws.numel(), _lib.stream(dev))
        return {s: e / draws for s, e in errors.items()}

    def reassemble(self, site, error):
        """The weight error of `site` from its output error (b, t, width) (dust.py:386-392): error times the captured
        input, summed over the tokens, [out, in] fp32; for the token embedding, the error rows added into their
        tokens' rows of a [padded vocab, 512] table."""
        if site not in self.inputs:
            raise KeyError(f'no linear input captured for site {site!r}')
        x = self.inputs[site]
        b, T = self.batch, self.length
        error = error.float().contiguous()
        if error.shape[:2] != (b, T):
            raise ValueError(f'error {tuple(error.shape)} does not match the captured batch ({b}, {T})')
        _lib.require_device(error)
        width = error.shape[-1]
        if site == 'transformer.wte':
            Vp = self.model.transformer.wte.weight.shape[0]
            out = torch.empty(Vp, width, dtype=torch.float32, device=error.device)
            _lib.call('noise_reassemble_embedding', _lib.ptr(error), width, _lib.ptr(x), b * T, Vp, width,
                      _lib.ptr(out), _lib.stream(error.device))
            return out
        d_in = x.shape[-1]
        out = torch.empty(width, d_in, dtype=torch.float32, device=error.device)
        _lib.call('noise_reassemble', _lib.ptr(error), width, _lib.ptr(x), int(x.dtype == torch.bfloat16), d_in, b * T,
                  width, d_in, 1.0, _lib.ptr(out), _lib.stream(error.device))
        return out
