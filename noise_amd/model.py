"""The fixed GPT of Noise with the reference's host API (utils/model.py), whose forward runs on the MI355X kernels.

GPTConfig, GPT(config, pad_vocab_size_to=64), init_weights(), forward(idx, targets=None, loss_reduction='mean') and
the state-dict keys, shapes and order are those of utils/model.py:34-210, so a state dict moves between the two
strictly (utils/eval.py:37-45). forward() calls the C-ABI population forward of libnoise_amd.so with one unperturbed
member per sequence; there is no CPU path, and a CPU tensor or a missing library raises.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch
from torch import nn
from torch.nn import functional as F

from . import _lib


@dataclass
class GPTConfig:
    sequence_len: int = 2048
    vocab_size: int = 4096
    n_layer: int = 8
    n_head: int = 8
    n_kv_head: int = 8
    n_embd: int = 512
    # Per block, repeating: S = half-sequence window, L = full. The last block is always L.
    window_pattern: str = 'SSSL'


def norm(x):
    return F.rms_norm(x, (x.size(-1),))


def has_ve(layer_idx, n_layer):
    """Value embeddings on every other block, counting back from the last (utils/model.py:50-52)."""
    return layer_idx % 2 == (n_layer - 1) % 2


def apply_rotary_emb(x, cos, sin):
    d = x.shape[3] // 2
    x1, x2 = x[..., :d], x[..., d:]
    return torch.cat([x1 * cos + x2 * sin, x1 * -sin + x2 * cos], 3)


def attention(q, k, v, window):
    """Causal attention with a left window on [batch, token, head, 64] tensors (utils/model.py:24-31): the HIP
    windowed flash kernel, bf16 operands, fp32 softmax statistics; the output in q's dtype. A length that is not a
    multiple of 128 is padded at the end (causal: the padding never reaches a real position)."""
    _lib.require_device(q, k, v)
    B, T, H, D = q.shape
    if D != 64:
        raise ValueError(f'head_dim must be 64, got {D}')
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f'q {tuple(q.shape)}, k {tuple(k.shape)} and v {tuple(v.shape)} must match')
    dtype = q.dtype
    Tp = (T + 127) // 128 * 128
    q, k, v = (F.pad(t.to(torch.bfloat16), (0, 0, 0, 0, 0, Tp - T)).contiguous() for t in (q, k, v))
    out = torch.empty_like(q)
    _lib.call('noise_attention', _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), B, H, Tp, Tp * H * D, H * D, int(window),
              _lib.ptr(out), Tp * H * D, H * D, None, _lib.stream(q.device))
    return out[:, :T].to(dtype)


def linear_bf16(x, weight):
    """x @ weight.t() as bf16 autocast computes it (bf16 operands, fp32 accumulation, bf16 output) on the HIP GEMM
    (noise_linear): x [..., in] on the GPU, weight [out, in] with in % 32 == 0 and out % 256 == 0."""
    _lib.require_device(x, weight)
    n_out, n_in = weight.shape
    lead = x.shape[:-1]
    xb = x.reshape(-1, n_in).to(torch.bfloat16).contiguous()
    wb = weight.detach().to(torch.bfloat16).contiguous()
    y = torch.empty(xb.shape[0], n_out, dtype=torch.bfloat16, device=x.device)
    if xb.shape[0]:
        _lib.call('noise_linear', _lib.ptr(xb), n_in, _lib.ptr(wb), xb.shape[0], n_in, n_out, _lib.ptr(y), n_out,
                  _lib.stream(x.device))
    return y.view(*lead, n_out)


class Linear(nn.Linear):
    """nn.Linear (same parameters and state-dict keys) whose bf16-autocast forward runs on the HIP GEMM: inside a
    cuda bf16 autocast region, with no autograd graph to record, y = bf16(x W^T) comes from noise_linear, as
    F.linear under autocast computes it. Elsewhere (fp32 calls, or a graph that needs gradients) it is nn.Linear."""

    def forward(self, x):
        if (x.is_cuda and self.bias is None and torch.is_autocast_enabled('cuda')
                and torch.get_autocast_dtype('cuda') == torch.bfloat16
                and self.in_features % 32 == 0 and self.out_features % 256 == 0
                and not (torch.is_grad_enabled() and (x.requires_grad or self.weight.requires_grad))):
            return linear_bf16(x, self.weight)
        return super().forward(x)


class CausalSelfAttention(nn.Module):
    def __init__(self, config, layer_idx):
        super().__init__()
        self.n_head = config.n_head
        self.n_kv_head = config.n_kv_head
        self.n_embd = config.n_embd
        self.head_dim = self.n_embd // self.n_head
        assert self.n_embd % self.n_head == 0
        self.c_q = Linear(self.n_embd, self.n_head * self.head_dim, bias=False)
        self.c_k = Linear(self.n_embd, self.n_kv_head * self.head_dim, bias=False)
        self.c_v = Linear(self.n_embd, self.n_kv_head * self.head_dim, bias=False)
        self.c_proj = Linear(self.n_embd, self.n_embd, bias=False)
        self.ve_gate_channels = 32
        self.ve_gate = (nn.Linear(self.ve_gate_channels, self.n_kv_head, bias=False)
                        if has_ve(layer_idx, config.n_layer) else None)

    def forward(self, x, ve, cos_sin, window_size):
        """utils/model.py:81-97 module by module (hooks on c_q, c_k, c_v, ve_gate and c_proj fire), the attention
        on the HIP flash kernel."""
        B, T, _ = x.shape
        q = self.c_q(x).view(B, T, self.n_head, self.head_dim)
        k = self.c_k(x).view(B, T, self.n_kv_head, self.head_dim)
        v = self.c_v(x).view(B, T, self.n_kv_head, self.head_dim)
        if ve is not None:
            gate = 2 * torch.sigmoid(self.ve_gate(x[..., :self.ve_gate_channels]))
            v = v + gate.unsqueeze(-1) * ve.view_as(v)
        cos, sin = cos_sin
        q, k = norm(apply_rotary_emb(q, cos, sin)), norm(apply_rotary_emb(k, cos, sin))
        return self.c_proj(attention(q, k, v, window_size[0]).reshape(B, T, -1))


class MLP(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.c_fc = Linear(config.n_embd, 4 * config.n_embd, bias=False)
        self.c_proj = Linear(4 * config.n_embd, config.n_embd, bias=False)

    def forward(self, x):
        """utils/model.py:106-107: c_proj(relu(c_fc(x))^2)."""
        return self.c_proj(F.relu(self.c_fc(x)).square())


class Block(nn.Module):
    def __init__(self, config, layer_idx):
        super().__init__()
        self.attn = CausalSelfAttention(config, layer_idx)
        self.mlp = MLP(config)

    def forward(self, x, ve, cos_sin, window_size):
        """utils/model.py:116-120: the pre-norm residual block."""
        x = x + self.attn(norm(x), ve, cos_sin, window_size)
        return x + self.mlp(norm(x))


def _hooked(model):
    """True when a forward hook or pre-hook sits on any submodule (or globally): the fused forward would skip it."""
    from torch.nn.modules import module as _m
    if _m._global_forward_hooks or _m._global_forward_pre_hooks:
        return True
    return any(m._forward_hooks or m._forward_pre_hooks for m in model.modules() if m is not model)


class GPT(nn.Module):
    def __init__(self, config, pad_vocab_size_to=64):
        super().__init__()
        self.config = config
        self.window_sizes = self._compute_window_sizes(config)
        padded_vocab = (config.vocab_size + pad_vocab_size_to - 1) // pad_vocab_size_to * pad_vocab_size_to
        self.transformer = nn.ModuleDict({
            'wte': nn.Embedding(padded_vocab, config.n_embd),
            'h': nn.ModuleList([Block(config, i) for i in range(config.n_layer)]),
        })
        self.lm_head = Linear(config.n_embd, padded_vocab, bias=False)
        self.resid_lambdas = nn.Parameter(torch.ones(config.n_layer))
        self.x0_lambdas = nn.Parameter(torch.zeros(config.n_layer))
        head_dim = config.n_embd // config.n_head
        kv_dim = config.n_kv_head * head_dim
        self.value_embeds = nn.ModuleDict({
            str(i): nn.Embedding(padded_vocab, kv_dim) for i in range(config.n_layer) if has_ve(i, config.n_layer)
        })
        self.rotary_seq_len = config.sequence_len * 10
        cos, sin = self._precompute_rotary(self.rotary_seq_len, head_dim)
        self.register_buffer('cos', cos, persistent=False)
        self.register_buffer('sin', sin, persistent=False)
        self._packed = None

    @torch.no_grad()
    def init_weights(self):
        """utils/model.py:149-175: N(0,1) wte, N(0,1e-3) lm_head, U(+-sqrt(3/512)) q/k/v/c_fc/value embeddings,
        zero c_proj and ve_gate, lambdas 1 and 0.1, bf16 rotary tables, bf16 embeddings on the GPU."""
        torch.nn.init.normal_(self.transformer.wte.weight, mean=0.0, std=1.0)
        torch.nn.init.normal_(self.lm_head.weight, mean=0.0, std=0.001)
        s = 3 ** 0.5 * self.config.n_embd ** (-0.5)
        for block in self.transformer.h:
            torch.nn.init.uniform_(block.attn.c_q.weight, -s, s)
            torch.nn.init.uniform_(block.attn.c_k.weight, -s, s)
            torch.nn.init.uniform_(block.attn.c_v.weight, -s, s)
            torch.nn.init.zeros_(block.attn.c_proj.weight)
            torch.nn.init.uniform_(block.mlp.c_fc.weight, -s, s)
            torch.nn.init.zeros_(block.mlp.c_proj.weight)
        self.resid_lambdas.fill_(1.0)
        self.x0_lambdas.fill_(0.1)
        for ve in self.value_embeds.values():
            torch.nn.init.uniform_(ve.weight, -s, s)
        for block in self.transformer.h:
            if block.attn.ve_gate is not None:
                torch.nn.init.zeros_(block.attn.ve_gate.weight)
        head_dim = self.config.n_embd // self.config.n_head
        self.cos, self.sin = self._precompute_rotary(self.rotary_seq_len, head_dim)
        if self.transformer.wte.weight.device.type == 'cuda':
            self.transformer.wte.to(dtype=torch.bfloat16)
            for ve in self.value_embeds.values():
                ve.to(dtype=torch.bfloat16)
        self._packed = None

    def _precompute_rotary(self, seq_len, head_dim, base=10000):
        device = self.transformer.wte.weight.device
        inv_freq = 1.0 / base ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim)
        t = torch.arange(seq_len, dtype=torch.float32, device=device)
        freqs = torch.outer(t, inv_freq)
        cos, sin = freqs.cos().bfloat16(), freqs.sin().bfloat16()
        return cos[None, :, None, :], sin[None, :, None, :]

    def _compute_window_sizes(self, config):
        pattern = config.window_pattern.upper()
        long_w, short_w = config.sequence_len, config.sequence_len // 2
        char_to_w = {'L': (long_w, 0), 'S': (short_w, 0)}
        sizes = [char_to_w[pattern[i % len(pattern)]] for i in range(config.n_layer)]
        sizes[-1] = (long_w, 0)
        return sizes

    # ---- device views for the kernels -----------------------------------------------------------------------
    def check_shape(self):
        c = self.config
        if (c.n_embd, c.n_head, c.n_kv_head) != (512, 8, 8):
            raise ValueError('the HIP kernels are built for the fixed model: n_embd 512, 8 heads of 64')
        if c.n_layer > _lib.MAX_LAYERS:
            raise ValueError(f'n_layer {c.n_layer} > {_lib.MAX_LAYERS}')
        if self.lm_head.weight.shape[0] % 256 or self.lm_head.weight.shape[0] > 4096:
            raise ValueError('padded vocabulary must be a multiple of 256 and at most 4096')

    def packed(self):
        """bf16 GEMM operands, fp32 tables and the ctypes model struct; rebuilt when any parameter changed."""
        params = list(self.parameters())
        key = tuple((p.data_ptr(), p._version) for p in params)
        if self._packed is not None and self._packed[0] == key:
            return self._packed[1]
        self.check_shape()
        dev = self.lm_head.weight.device
        _lib.require_device(self.lm_head.weight)
        keep = {}
        bf = lambda t: t.detach().to(torch.bfloat16).contiguous()
        f32 = lambda t: t.detach().to(torch.float32).contiguous()
        s = _lib.NoiseGpt()
        s.n_layer = self.config.n_layer
        s.vocab = self.config.vocab_size
        s.padded_vocab = self.lm_head.weight.shape[0]
        keep['resid'] = f32(self.resid_lambdas)
        keep['x0l'] = f32(self.x0_lambdas)
        keep['wte'] = f32(self.transformer.wte.weight)
        keep['lm_head'] = bf(self.lm_head.weight)
        s.resid_lambdas, s.x0_lambdas = keep['resid'].data_ptr(), keep['x0l'].data_ptr()
        s.wte, s.lm_head = keep['wte'].data_ptr(), keep['lm_head'].data_ptr()
        for i, block in enumerate(self.transformer.h):
            a, m = block.attn, block.mlp
            L = s.layers[i]
            keep[f'qkv{i}'] = bf(torch.cat([a.c_q.weight, a.c_k.weight, a.c_v.weight]))
            keep[f'proj{i}'] = bf(a.c_proj.weight)
            keep[f'fc{i}'] = bf(m.c_fc.weight)
            keep[f'mproj{i}'] = bf(m.c_proj.weight)
            L.w_qkv, L.w_proj = keep[f'qkv{i}'].data_ptr(), keep[f'proj{i}'].data_ptr()
            L.w_fc, L.w_mlp_proj = keep[f'fc{i}'].data_ptr(), keep[f'mproj{i}'].data_ptr()
            if a.ve_gate is not None:
                keep[f'gate{i}'] = f32(a.ve_gate.weight)
                keep[f've{i}'] = f32(self.value_embeds[str(i)].weight)
                L.w_gate, L.ve = keep[f'gate{i}'].data_ptr(), keep[f've{i}'].data_ptr()
            L.window = int(self.window_sizes[i][0])
        self._packed = (key, (s, keep, dev))
        return self._packed[1]

    def rope_tables(self, T):
        cos = self.cos[0, :T, 0, :].float().contiguous()
        sin = self.sin[0, :T, 0, :].float().contiguous()
        return cos, sin

    def forward(self, idx, targets=None, loss_reduction='mean'):
        """utils/model.py:193-210 on the HIP kernels: logits fp32 [B, T, vocab] (soft-capped) without targets,
        otherwise the cross-entropy ('mean' over targets != -1, 'sum', or 'none' [B * T]).

        The fused population forward computes the whole model in a few kernels and never calls the submodules. When
        a caller has registered hooks on submodules (Dust's capture does, train/val/dust.py:166-168), the forward
        runs module by module instead, under bf16 autocast, so every hook sees its module's input and output."""
        _lib.require_device(idx)
        if _hooked(self):
            return self._forward_modules(idx, targets, loss_reduction)
        B, T = idx.shape
        Tp = (T + 127) // 128 * 128
        idx = idx.to(torch.int64)
        if Tp != T:  # causal: trailing padding does not reach the real positions
            idx = F.pad(idx, (0, Tp - T))
        tg = None
        if targets is not None:
            tg = targets.to(torch.int64)
            if Tp != T:
                tg = F.pad(tg, (0, Tp - T), value=-1)
            tg = tg.contiguous()
        from .population import run_forward
        out = run_forward(self, idx.contiguous(), tg, member_seq=torch.arange(B, device=idx.device, dtype=torch.int32),
                          noise=None, want_logits=targets is None, want_tokens=loss_reduction == 'none',
                          check_tables=False)
        if targets is None:
            return out['logits'].view(B, Tp, -1)[:, :T]
        if loss_reduction == 'none':
            return out['token_loss'].view(B, Tp)[:, :T].reshape(-1)
        total = out['loss_sum'].sum()
        if loss_reduction == 'sum':
            return total
        if loss_reduction == 'mean':
            return total / (targets != -1).sum()
        raise ValueError(f'unknown loss_reduction {loss_reduction!r}')

    def _forward_modules(self, idx, targets, loss_reduction):
        """The module-by-module forward (utils/model.py:193-210's call sequence, which hooks observe): the bf16
        linears on the HIP GEMM (Linear, noise_linear; the 32 -> 8 value-embedding gate on torch's), the HIP flash
        attention, and torch's elementwise ops under bf16 autocast as the reference's."""
        B, T = idx.shape
        cos_sin = (self.cos[:, :T], self.sin[:, :T])
        with torch.autocast('cuda', dtype=torch.bfloat16):
            x0 = x = norm(self.transformer.wte(idx))
            for i, block in enumerate(self.transformer.h):
                x = self.resid_lambdas[i] * x + self.x0_lambdas[i] * x0
                ve = self.value_embeds[str(i)](idx) if str(i) in self.value_embeds else None
                x = block(x, ve, cos_sin, self.window_sizes[i])
            logits = self.lm_head(norm(x))[..., :self.config.vocab_size].float()
        logits = 15 * torch.tanh(logits / 15)
        if targets is None:
            return logits
        return F.cross_entropy(logits.reshape(-1, logits.shape[-1]), targets.reshape(-1), ignore_index=-1,
                               reduction=loss_reduction)
