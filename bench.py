#!/usr/bin/env python3
"""Benchmark of the population hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload c4|c5] [--no-cpu-baseline] [--no-credit] [--no-dust]
    python bench.py --copy-calibration      # one plain 1 GiB device copy, to scale rocprofv3 FETCH/WRITE_SIZE

A step is one pass of the hot path over one batch of synthetic input:
  c4 (default): the 8-layer population forward of config 4: 256 antithetic members (128 pairs), each
      evaluating 2 sequences x 2048 Zipf(1.1) tokens over vocab 4096, weights N(0, 0.02) (lambdas 1 / 0.1), with the
      per-step noise offsets and rows generated on the GPU; output per-member summed CE. 1,048,576 member-tokens.
  c5: one full EGGROLL training step (config 5): 12,288 pairs = 24,576 members over an 8 x 2048 batch, chunks of
      512 members, fitness, outer-product gradient assembly and AdamW. 50,331,648 member-tokens.
The JSON line carries the headline metric (member-tokens/s), the roofline of the dominant kernel (HIP events on the launch
stream over the timed region), the oracle's CPU throughput on a bounded sample, the credit readout's TFLOP/s at
config 3 (B16 H8 T2048 d64), and the time of Dust's head-slab estimator, of one group of its direct draws and of one
whole Dust update at the reference recipe's per-GPU draw counts. `roofline.traffic` is the dominant kernel's HBM bytes per launch as recorded in
profiles/population_forward_c4_traffic.txt (rocprofv3 FETCH_SIZE and WRITE_SIZE passes over this script, each scaled
by what the counter reads for --copy-calibration); it is null for a workload or kernel that file does not cover.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

METRIC = 'perturbed-forward tokens/sec (members×tokens) at 37.7M; credit kernel TFLOP/s'
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
PEAK_FP32_TFLOPS = 157.3
FLOP_PER_MEMBER_TOKEN = 68.170752e6
D, F, QKV, V, T_SEQ = 512, 2048, 1536, 4096, 2048


def zipf_tokens(n_rows, T, seed, vocab=V, s=1.1):
    import torch
    p = (torch.arange(vocab, dtype=torch.float64) + 1.0) ** -s
    cdf = torch.cumsum(p / p.sum(), 0)
    u = torch.rand(n_rows, T + 1, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)
    rows = torch.searchsorted(cdf, u).clamp(max=vocab - 1)
    return rows[:, :-1].contiguous(), rows[:, 1:].contiguous()


def make_model(dev, seed=0, n_layer=8):
    import torch
    from noise_amd.model import GPT, GPTConfig
    torch.manual_seed(seed)
    with torch.device('meta'):
        model = GPT(GPTConfig(n_layer=n_layer))
    model.to_empty(device=dev)
    model.init_weights()
    model.transformer.wte.float()
    for e in model.value_embeds.values():
        e.float()
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.dim() == 2:
                p.normal_(0.0, 0.02)
    return model.requires_grad_(False)


def attention_flops(members_rows, windows, T):
    tot = 0.0
    for w in windows:
        keys = sum(min(t, w) + 1 for t in range(T))
        tot += 4 * D * keys
    return tot * members_rows  # members_rows = evaluations (rows of T tokens)


def kernel_flops(n_eval, T, windows, n_layer):
    """Algorithmic FLOPs per launch of each timed kernel class (rank-1 terms excluded, in-window pairs only)."""
    M = n_eval * T
    return {
        'qkv_gemm': 2.0 * M * QKV * D,
        'attn_proj_gemm': 2.0 * M * D * D,
        'fc_gemm': 2.0 * M * F * D,
        'mlp_proj_gemm': 2.0 * M * D * F,
        'head_ce_gemm': 2.0 * M * V * D,
        'attention': attention_flops(n_eval, windows, T) / n_layer,
    }


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'profiles', 'population_forward_c4_traffic.txt')


def load_traffic(path=TRAFFIC_FILE):
    """Per-class HBM bytes per launch from the committed rocprofv3 summary: lines `traffic <class> <bytes> ...`."""
    out = {}
    if not os.path.exists(path):
        return out
    with open(path) as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 3 and parts[0] == 'traffic':
                out[parts[1]] = int(parts[2])
    return out


def roofline_from_timing(timing, flops, traffic=None):
    kernels = {}
    for name, f in flops.items():
        n, ms = timing.get(name, (0, 0.0))
        if n == 0:
            continue
        avg_ms = ms / n
        tf = f / (avg_ms * 1e-3) / 1e12
        kernels[name] = dict(launches=n, avg_ms=round(avg_ms, 4), total_ms=round(ms, 3), tflops=round(tf, 1),
                             frac=round(tf / PEAK_BF16_TFLOPS, 4))
    for name, (n, ms) in timing.items():
        if n and name not in kernels:
            kernels[name] = dict(launches=n, avg_ms=round(ms / n, 4), total_ms=round(ms, 3))
    dom = max(flops.keys() & kernels.keys(), key=lambda k: kernels[k]['total_ms'])
    k = kernels[dom]
    roof = dict(bound='mfma', kernel=dom, achieved=k['tflops'], peak=PEAK_BF16_TFLOPS, unit='TFLOP/s', frac=k['frac'],
                traffic=(traffic or {}).get(dom), flop_per_launch=flops[dom], avg_launch_ms=k['avg_ms'])
    if roof['traffic'] is not None:
        roof['traffic_source'] = 'profiles/' + os.path.basename(TRAFFIC_FILE)
        roof['traffic_gbs'] = round(roof['traffic'] / (k['avg_ms'] * 1e-3) / 1e9, 1)
    return roof, kernels


def bench_c4(args, dev, n_layer=8):
    import torch
    from noise_amd import _lib
    from noise_amd.population import Eggroll, NoiseLayout, run_forward
    model = make_model(dev, n_layer=n_layer)
    pairs, n_seq = 128, 2
    members = 2 * pairs
    x, y = zipf_tokens(n_seq, T_SEQ, seed=0)
    x, y = x.to(dev), y.to(dev)
    es = Eggroll(model, pairs, sigma=0.002, seed=0)
    layout = NoiseLayout(model)
    # evaluation e = (member e // 2, sequence e % 2): the member's pair direction and antithetic sign
    ev = torch.arange(members * n_seq, device=dev)
    member = ev // n_seq
    member_seq = (ev % n_seq).to(torch.int32)
    member_row = (member // 2).to(torch.int32)
    member_sign = torch.where(member % 2 == 0, 0.002, -0.002).float()
    all_dirs = torch.arange(pairs, device=dev)

    def step(i):
        table = es.offset_table(i)
        rows = es.rows(table, all_dirs)
        out = run_forward(model, x, y, member_seq, noise=rows, member_row=member_row, member_sign=member_sign,
                          layout=layout, check_tables=False)
        return out['loss_sum'].view(members, n_seq).sum(1)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    _lib.timing_enable(True)
    t0 = time.perf_counter()
    for i in range(args.steps):
        losses = step(args.warmup + i)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    timing = _lib.timing_read()
    _lib.timing_enable(False)
    finite = bool(torch.isfinite(losses).all().item())
    member_tokens = members * n_seq * T_SEQ
    windows = [w for w, _ in model.window_sizes]
    roof, kernels = roofline_from_timing(timing, kernel_flops(members * n_seq, T_SEQ, windows, len(windows)),
                                         load_traffic())
    flops = kernel_flops(members * n_seq, T_SEQ, windows, len(windows))
    step_flop = len(windows) * sum(flops[k] for k in ('qkv_gemm', 'attn_proj_gemm', 'fc_gemm', 'mlp_proj_gemm',
                                                      'attention')) + flops['head_ce_gemm']
    res = dict(value=member_tokens * args.steps / dt, ms_per_step=dt / args.steps * 1e3, member_tokens=member_tokens,
               roofline=roof, kernels=kernels, finite=finite, step_flop=step_flop,
               mean_member_ce=float(losses.mean().item() / (n_seq * T_SEQ)),
               config=dict(workload=f'C4: {len(windows)}-layer population forward, 256 antithetic members (128 '
                           'pairs) x 2 sequences x 2048 Zipf(1.1) tokens, vocab 4096, N(0,0.02) weights, in-kernel '
                           'counter noise',
                           members=members, sequences_per_member=n_seq, seq_len=T_SEQ, n_layer=len(windows),
                           params=sum(p.numel() for p in model.parameters()), parallelism='single GPU'))
    res['model'] = model
    return res


def bench_c5(args, dev, steps=None, warmup=None):
    import torch
    from noise_amd import _lib
    from noise_amd.optim import AdamW
    from noise_amd.population import Eggroll
    model = make_model(dev)
    pairs, n_seq = 12288, 8
    x, y = zipf_tokens(n_seq, T_SEQ, seed=0)
    x, y = x.to(dev), y.to(dev)
    es = Eggroll(model, pairs, sigma=0.002, seed=0, chunk=256)
    opt = AdamW(model.parameters(), lr=1e-3, betas=(0.5, 0.95), eps=1e-8, weight_decay=0.0)
    # the step's credit readout over the clean batch (B 8, 8 heads, 8 layers, T window): per-token error signals of
    # dim 64 credited through each layer's q / k (synthetic, as config 3's)
    from noise_amd import credit
    g = torch.Generator(device=dev).manual_seed(1)
    cq = (torch.randn(n_seq * 8, T_SEQ, 64, device=dev, generator=g) / 8).bfloat16()
    ck = (torch.randn(n_seq * 8, T_SEQ, 64, device=dev, generator=g) / 8).bfloat16()
    ce = torch.randn(n_seq * 8, T_SEQ, 64, device=dev, generator=g)
    n_layer = model.config.n_layer
    if (cq.float().norm(dim=-1).max() * ck.float().norm(dim=-1).max()).item() / 8 > 16:
        raise RuntimeError('c5 bench: the credit logits exceed the bounded LSE pass\'s 16')

    def step(i):
        loss = es.step(x, y, opt, i)
        for _ in range(n_layer):
            credit.value_credit(cq, ck, ce, T_SEQ, hi_lo=False, bounded=True)
        return loss

    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    for i in range(warmup):
        step(i + 1)
    torch.cuda.synchronize()
    _lib.timing_enable(True)
    t0 = time.perf_counter()
    for i in range(steps):
        loss = step(warmup + i + 1)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    timing = _lib.timing_read()
    _lib.timing_enable(False)
    members = 2 * pairs
    member_tokens = members * T_SEQ
    windows = [w for w, _ in model.window_sizes]
    roof, kernels = roofline_from_timing(timing, kernel_flops(2 * es.chunk, T_SEQ, windows, len(windows)))
    n_params = sum(p.numel() for p in model.parameters())
    mat_params = sum(p.numel() for p in model.parameters() if p.dim() == 2)
    per_step = lambda name: timing.get(name, (0, 0.0))[1] / steps
    adam_ms, og_ms = per_step('adamw'), per_step('outer_grad')
    update = dict(
        fitness_ms=round(per_step('fitness'), 4), vector_grad_ms=round(per_step('vector_grad'), 4),
        outer_grad_ms=round(og_ms, 3),
        outer_grad_tflops=round(2.0 * mat_params * pairs / (og_ms * 1e-3) / 1e12, 1) if og_ms else None,
        outer_grad_note='fp32 MFMA products over K = 12,288 pairs (0.93 TFLOP); peak 157.3 TFLOP/s fp32',
        adamw_ms=round(adam_ms, 4), adamw_bytes=28 * n_params,
        adamw_gbs=round(28 * n_params / (adam_ms * 1e-3) / 1e9, 1) if adam_ms else None,
        adamw_hbm_frac=round(28 * n_params / (adam_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4) if adam_ms else None,
        noise_rows_ms=round(per_step('noise'), 3))
    fwd_classes = ('embed', 'qkv_gemm', 'attention', 'attn_proj_gemm', 'fc_gemm', 'mlp_proj_gemm', 'head_ce_gemm',
                   'ce_finalize', 'norm')
    fwd_ms = sum(per_step(c) for c in fwd_classes)
    res = dict(value=member_tokens * steps / dt, ms_per_step=dt / steps * 1e3, member_tokens=member_tokens,
               update=update, forward_kernels_ms=round(fwd_ms, 2),
               credit_ms=round(per_step('credit_lse') + per_step('credit_value'), 3),
               roofline=roof, kernels=kernels, finite=math.isfinite(loss), mean_member_ce=loss,
               config=dict(workload='C5: full EGGROLL step, 24,576 members (12,288 pairs) in chunks of 512 over an '
                           '8 x 2048 Zipf(1.1) batch, fitness, outer-product gradients, AdamW, and the credit readout '
                           'over the clean batch (8 layers x B8 H8 T2048, synthetic q / k / error signals)',
                           members=members, seq_len=T_SEQ, n_layer=len(windows), parallelism='single GPU'))
    res['model'] = model
    return res


def bench_hooked_forward(dev, model, iters=5):
    """GPT.forward (utils/model.py:193-210) on an 8 x 2048 Zipf(1.1) batch two ways: the fused population forward
    (one unperturbed member per sequence), and module by module, as it runs when a caller hooks submodules
    (train/val/dust.py:166-168): the linears on noise_linear, the attention on the flash kernel, torch's elementwise
    ops under bf16 autocast. Each a median of `iters` timed calls after one warmup, no autograd."""
    import torch
    from noise_amd import _lib
    x, y = zipf_tokens(8, T_SEQ, seed=3)
    x, y = x.to(dev), y.to(dev)
    out = {}
    for name, hooked in (('fused', False), ('hooked', True)):
        h = model.lm_head.register_forward_hook(lambda *a: None) if hooked else None
        try:
            with torch.no_grad():
                model(x, y)
                torch.cuda.synchronize()
                _lib.timing_enable(True)
                times = []
                for _ in range(iters):
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    loss = model(x, y)
                    e1.record()
                    torch.cuda.synchronize()
                    times.append(e0.elapsed_time(e1))
                tm = _lib.timing_read()
                _lib.timing_enable(False)
        finally:
            if h is not None:
                h.remove()
        ms = statistics.median(times)
        out[name] = dict(ms=round(ms, 3), tokens_per_s=round(8 * T_SEQ / (ms * 1e-3), 1),
                         loss=round(float(loss), 4))
        if hooked:
            n, lin_ms = tm.get('linear', (0, 0.0))
            out[name]['linear_launches_per_call'] = n // iters
            out[name]['linear_ms_per_call'] = round(lin_ms / iters, 3)
    out['note'] = ('8 x 2048 tokens, no perturbation; hooked: a no-op forward hook on lm_head sends GPT.forward '
                   'module by module (the reference\'s call sequence), its linears on noise_linear')
    return out


def c4_12layer_record(dev, steps=5, warmup=1):
    """BASELINE.json's configs[3] read literally: the config-4 population forward on the 12-layer model (GPTConfig
    n_layer=12, 54.5M parameters; windows SSSL repeated, value embeddings on alternate layers), same members, tokens
    and noise as the headline, fewer steps."""
    import types
    res = bench_c4(types.SimpleNamespace(steps=steps, warmup=warmup), dev, n_layer=12)
    res.pop('model')
    tf = res['step_flop'] / (res['ms_per_step'] * 1e-3) / 1e12
    return dict(workload=res['config']['workload'], n_layer=12, params=res['config']['params'], steps=steps,
                warmup=warmup, ms_per_step=round(res['ms_per_step'], 3),
                member_tokens_per_s=round(res['value'], 1),
                flop_per_member_token=round(res['step_flop'] / res['member_tokens'], 1),
                forward_tflops=round(tf, 1), forward_frac=round(tf / PEAK_BF16_TFLOPS, 4), finite=res['finite'],
                kernels={k: dict(avg_ms=v['avg_ms'], tflops=v.get('tflops')) for k, v in res['kernels'].items()
                         if 'tflops' in v})


def c5_record(dev):
    """Config 5 in the default run: 1 warmup step, then 2 timed steps, each a full EGGROLL update."""
    import types
    res = bench_c5(types.SimpleNamespace(steps=2, warmup=1), dev, steps=2, warmup=1)
    res.pop('model')
    fwd = res['value'] * FLOP_PER_MEMBER_TOKEN / 1e12
    return dict(workload=res['config']['workload'], steps=2, warmup=1, ms_per_step=round(res['ms_per_step'], 1),
                member_tokens_per_s=round(res['value'], 1), forward_equivalent_tflops=round(fwd, 1),
                forward_frac=round(fwd / PEAK_BF16_TFLOPS, 4), forward_kernels_ms=res['forward_kernels_ms'],
                update=res['update'], credit_readout_ms=res['credit_ms'], finite=res['finite'],
                target_ms_per_step=2270.0)


def bench_credit(dev, iters=10):
    """Config 3: lse + value pass, B16 H8 T2048 d64, Q/K bf16 N(0,1)/8, E N(0,1) fp32, full causal window and 1024;
    also the key-context pass (lse and center) on the same q / k with bf16 values and hub. The LSE pass runs its
    bounded form (no running maximum), after a check that max|q| max|k| / 8, a bound on every logit, is <= 16."""
    import torch
    from noise_amd import _lib, credit
    rows, T = 16 * 8, 2048
    g = torch.Generator(device=dev).manual_seed(0)
    q = (torch.randn(rows, T, 64, device=dev, generator=g) / 8).bfloat16()
    k = (torch.randn(rows, T, 64, device=dev, generator=g) / 8).bfloat16()
    e = torch.randn(rows, T, 64, device=dev, generator=g)
    pairs = rows * T * (T + 1) // 2
    logit_bound = (q.float().norm(dim=-1).max() * k.float().norm(dim=-1).max()).item() / 8  # Cauchy-Schwarz
    if logit_bound > 16:
        raise RuntimeError(f'credit bench: logits up to {logit_bound:.1f} exceed the bounded LSE pass\'s 16')
    out = {'logit_bound': round(logit_bound, 3)}
    for window in (T, 1024):
        npairs = rows * sum(min(t, window) + 1 for t in range(T))
        flops = 6 * 64 * npairs
        for hi_lo in (False, True):  # the speedrun's production setting (value_gluon HI = 1), then high + low
            for _ in range(2):
                credit.value_credit(q, k, e, window, hi_lo=hi_lo, bounded=True)
            torch.cuda.synchronize()
            _lib.timing_enable(True)
            for _ in range(iters):
                credit.value_credit(q, k, e, window, hi_lo=hi_lo, bounded=True)
            torch.cuda.synchronize()
            tm = _lib.timing_read()
            _lib.timing_enable(False)
            lse_ms = tm['credit_lse'][1] / tm['credit_lse'][0]
            val_ms = tm['credit_value'][1] / tm['credit_value'][0]
            if not hi_lo:
                out[f'window_{window}'] = dict(
                    pairs=npairs, tflops=round(flops / ((lse_ms + val_ms) * 1e-3) / 1e12, 1),
                    frac=round(flops / ((lse_ms + val_ms) * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                    lse_ms=round(lse_ms, 4), value_ms=round(val_ms, 4),
                    value_pass_tflops=round(4 * 64 * npairs / (val_ms * 1e-3) / 1e12, 1),
                    source='bf16 high part (the speedrun\'s HI = 1)')
            else:
                out[f'window_{window}'].update(hi_lo_value_ms=round(val_ms, 4),
                                               hi_lo_tflops=round(flops / ((lse_ms + val_ms) * 1e-3) / 1e12, 1))
        # the general readout: the LSE pass with its running maximum (no bound on the logits, as the reference's
        # kernels), then the same value pass
        for _ in range(2):
            credit.value_credit(q, k, e, window, hi_lo=False, bounded=False)
        torch.cuda.synchronize()
        _lib.timing_enable(True)
        for _ in range(iters):
            credit.value_credit(q, k, e, window, hi_lo=False, bounded=False)
        torch.cuda.synchronize()
        tm = _lib.timing_read()
        _lib.timing_enable(False)
        rm_lse = tm['credit_lse'][1] / tm['credit_lse'][0]
        rm_val = tm['credit_value'][1] / tm['credit_value'][0]
        out[f'window_{window}'].update(running_max_lse_ms=round(rm_lse, 4), running_max_value_ms=round(rm_val, 4),
                                       running_max_tflops=round(flops / ((rm_lse + rm_val) * 1e-3) / 1e12, 1))
        # the key-context pass (lse and center): q.k and hub.v dots, 4d FLOPs per pair
        vals = (torch.randn(rows, T, 64, device=dev, generator=g)).bfloat16()
        hub = e.bfloat16()
        for _ in range(2):
            credit.key_context(q, k, vals, hub, window)
        torch.cuda.synchronize()
        _lib.timing_enable(True)
        for _ in range(iters):
            credit.key_context(q, k, vals, hub, window)
        torch.cuda.synchronize()
        tm = _lib.timing_read()
        _lib.timing_enable(False)
        ctx_ms = tm['credit_center'][1] / tm['credit_center'][0]
        out[f'window_{window}'].update(key_context_ms=round(ctx_ms, 4),
                                       key_context_tflops=round(4 * 64 * npairs / (ctx_ms * 1e-3) / 1e12, 1))
    out['headline'] = f"{out[f'window_{T}']['tflops']} TFLOP/s at 6d per causal pair ({pairs:,} pairs)"
    return out


def bench_c2(dev, iters=20):
    """Config 2: the single perturbed linear, X bf16 [32768, 512] N(0, 1) shared by 64 members (32 antithetic pairs,
    sigma 1e-3), W [2048, 512] N(0, 0.02), a_i and b_i N(0, 1) from the counter generator; per-member sums of squares
    of y_i = X W^T + s_i (X b_i) a_i^T, y never stored. Both evaluations: the expanded square (member terms on the
    MFMA units) and every element formed (2 fp32 FMAs per element and member)."""
    import torch
    from noise_amd import _lib
    from noise_amd.population import lowrank_sumsq
    T, n_in, n_out, m, sigma = 32768, 512, 2048, 64, 1e-3
    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn(T, n_in, device=dev, generator=g).bfloat16()
    W = (torch.randn(n_out, n_in, device=dev, generator=g) * 0.02).bfloat16()
    rows = torch.empty(m, n_out + n_in, device=dev)
    _lib.call('noise_rng_buffer', 0, 0, rows.numel(), _lib.ptr(rows), _lib.stream(dev))
    sign = torch.tensor([sigma if i % 2 == 0 else -sigma for i in range(m)], device=dev)
    member_tokens = m * T
    gemm_flop = 2.0 * T * n_in * n_out
    xb_flop = 2.0 * m * T * n_in
    epi_flop = 4.0 * m * T * n_out  # rank-1 apply (2) and square-accumulate (2) per element and member
    out = dict(workload='C2: X [32768, 512] bf16 shared by 64 members (32 pairs, sigma 1e-3), W [2048, 512]; '
               'per-member sum of squares of the [64, 32768, 2048] outputs, y never stored',
               member_tokens=member_tokens, algorithmic_gflop=round((gemm_flop + xb_flop + epi_flop) / 1e9, 2),
               shared_gemm_gflop=round(gemm_flop / 1e9, 2), epilogue_gflop=round(epi_flop / 1e9, 2))
    for mode in ('expansion', 'direct'):
        for _ in range(3):
            s = lowrank_sumsq(x, W, rows, 0, n_out, sign, mode=mode)
        torch.cuda.synchronize()
        _lib.timing_enable(True)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            s = lowrank_sumsq(x, W, rows, 0, n_out, sign, mode=mode)
        e1.record()
        torch.cuda.synchronize()
        tm = _lib.timing_read()
        _lib.timing_enable(False)
        call_ms = e0.elapsed_time(e1) / iters
        gemm_ms = tm['lowrank_gemm'][1] / tm['lowrank_gemm'][0]
        rec = dict(
            ms_per_call=round(call_ms, 4), member_tokens_per_s=round(member_tokens / (call_ms * 1e-3), 1),
            gemm_kernel_ms=round(gemm_ms, 4), pre_ms=round(tm['lowrank_pre'][1] / tm['lowrank_pre'][0], 4),
            finish_ms=round(tm['lowrank_post'][1] / tm['lowrank_post'][0], 4),
            algorithmic_tflops=round((gemm_flop + xb_flop + epi_flop) / (call_ms * 1e-3) / 1e12, 1),
            mfma_frac=round(gemm_flop / (gemm_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            finite=bool(torch.isfinite(s).all()))
        if mode == 'direct':  # the per-element epilogue runs on the fp32 VALU
            rec['valu_frac'] = round(epi_flop / (gemm_ms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS, 4)
        else:  # the member terms run on the MFMA units: E_i = u_i^T C per tile, 2 T N FLOP per member
            member_flop = 2.0 * m * T * n_out
            rec['member_mfma_gflop'] = round(member_flop / 1e9, 2)
            rec['mfma_frac_with_member_terms'] = round((gemm_flop + member_flop) / (gemm_ms * 1e-3) / 1e12
                                                       / PEAK_BF16_TFLOPS, 4)
        out[mode] = rec
    out['note'] = ('mfma_frac: the 68.72 GFLOP shared GEMM over the fused kernel\'s mean launch. direct: every '
                   'element formed, valu_frac = the 17.18 GFLOP rank-1 apply and square-accumulate over the same '
                   'launch against the 157.3 TFLOP/s fp32 vector peak (which counts packed fp32; this build compiles '
                   'packed fp32 off, so 78.6 TFLOP/s is its ceiling). expansion: the member work is 8.59 GFLOP of '
                   'MFMA products on the accumulator tiles instead, and no per-element VALU pass')
    return out


def bench_head_error(dev, iters=3):
    """Dust's head-slab CE estimator (train/val/dust.py:261-303) at the reference recipe's per-GPU head draws
    (recipe(1.5).head = 73,728 over 8 GPUs = 9,216, nrep 16) over an 8 x 2048 token batch, vocabulary 4096."""
    import torch
    from noise_amd import _lib, dust
    b, t, V, draws = 8, 2048, 4096, 9216
    g = torch.Generator(device=dev).manual_seed(0)
    raw = (3.0 * torch.randn(b, t, V, device=dev, generator=g)).bfloat16()
    y = torch.randint(0, V, (b, t), device=dev, generator=g)
    clean = 8.0 + torch.randn(b, t, device=dev, generator=g)
    dust.head_error(raw, y, clean, draws, sigma=0.1, nrep=16)
    torch.cuda.synchronize()
    _lib.timing_enable(True)
    for _ in range(iters):
        err = dust.head_error(raw, y, clean, draws, sigma=0.1, nrep=16)
    torch.cuda.synchronize()
    tm = _lib.timing_read()
    _lib.timing_enable(False)
    ms = tm['head_error'][1] / tm['head_error'][0]
    jittered = draws * b * t * 256
    return dict(ms=round(ms, 3), draws=draws, token_rows=b * t, vocab=V, finite=bool(torch.isfinite(err).all()),
                jittered_logits_per_s=round(jittered / (ms * 1e-3), 1),
                note='per call: 9,216 draws x 16,384 token rows x one 256-column slab, the jitter regenerated '
                     'twice from the counter stream (loss, then error), never stored')


def bench_dust_direct(dev, model, iters=2):
    """Dust's direct draws (train/val/dust.py:195-259) at the reference recipe's per-GPU counts: one direct_errors
    call for block 0's writers (attn.c_proj and mlp.c_proj outputs jittered together; recipe(1.5).writers = 384 draws
    over 8 GPUs = 48, chunks of nrep 16) on the 8 x 2048 batch; every draw reruns all 8 blocks."""
    import torch
    from noise_amd import _lib
    from noise_amd.dust import Dust
    x, y = zipf_tokens(8, T_SEQ, seed=1)
    x, y = x.to(dev), y.to(dev)
    d = Dust(model, nrep=16)
    d.capture(x, y)
    sites = ['transformer.h.0.attn.c_proj', 'transformer.h.0.mlp.c_proj']
    d.direct_errors(sites, 16, 0.4, entry=0)
    torch.cuda.synchronize()
    _lib.timing_enable(True)
    t0 = time.perf_counter()
    for _ in range(iters):
        err = d.direct_errors(sites, 48, 0.4, entry=0)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / iters
    tm = _lib.timing_read()
    _lib.timing_enable(False)
    member_tokens = 48 * 8 * T_SEQ
    return dict(ms=round(dt * 1e3, 2), draws=48, sequences=8, seq_len=T_SEQ,
                rerun_ms=round(tm['dust_rerun'][1] / iters, 2), errors_ms=round(tm['dust_errors'][1] / iters, 2),
                rerun_member_tokens_per_s=round(member_tokens / (tm['dust_rerun'][1] / iters * 1e-3), 1),
                finite=all(bool(torch.isfinite(e).all()) for e in err.values()))


def bench_dust_step(dev, steps=1):
    """One Dust update (train/val/dust.py:414-463) at one GPU's share of the reference's default recipe (recipe(1.5),
    every draw count / 8, as each of the reference's 8 GPUs runs it) on an 8 x 2048 Zipf batch of the reference's Dust
    model (make_model: c_proj uniform at 1.5 sqrt(3 / fan_in)), with the recipe's optimizer. The reference logs
    19,004.39 s for 1,831 updates on 8 H100s (train/val/dust_log/result.json): 10.38 s per update, each GPU doing
    this share. Phases: the direct draws (writers, hidden, embedding, attention outputs), the head slabs, the local
    draws of each kind with their reassembly, the mixing scalars."""
    import torch
    from noise_amd import dust as nd
    full = nd.recipe(1.5)
    w = 8
    r = nd.Recipe(writers=[c // w for c in full.writers], hidden=[c // w for c in full.hidden],
                  hubs=[c // w for c in full.hubs], embedding=full.embedding // w, head=full.head // w,
                  local={k: v // w for k, v in full.local.items()}, nrep=full.nrep, lr=full.lr, betas=full.betas,
                  warmdown=full.warmdown)
    model = nd.make_model(dev, 0)
    opt = nd.make_optimizer(model, r)
    d = nd.Dust(model, seed=0, recipe=r)
    x, y = zipf_tokens(8, T_SEQ, seed=3)
    x, y = x.to(dev), y.to(dev)

    def tick():
        torch.cuda.synchronize()
        return time.perf_counter()

    d.step(x, y, opt)  # warmup
    t0 = tick()
    for _ in range(steps):
        loss = d.step(x, y, opt)
    dt = (tick() - t0) / steps
    # the phases of one more update's estimates, timed separately (the calls gradients() makes, in its order)
    phases = {}
    t = tick()
    d.capture(x, y)
    L = model.config.n_layer
    for layer in range(L):
        pre = f'transformer.h.{layer}.'
        gam = r.first_gamma if layer == 0 else 0.0
        for sites, count in [([pre + 'attn.c_proj', pre + 'mlp.c_proj'], r.writers[layer]),
                             ([pre + 'mlp.c_fc'], r.hidden[layer])]:
            for s_, e in d.direct_errors(sites, count, 0.4, layer, gam).items():
                d.reassemble(s_, e)
    phases['direct_writers_hidden_s'] = tick() - t
    t = tick()
    d.reassemble('transformer.wte', d.direct_errors(['transformer.wte'], r.embedding, 0.8)['transformer.wte'])
    phases['direct_embedding_s'] = tick() - t
    t = tick()
    targets = {i: d.direct_errors([f'o@{i}'], r.hubs[i], 0.4 if i < L // 2 else 0.8, i,
                                  r.first_gamma if i == 0 else 0.0)[f'o@{i}'] for i in range(L)}
    phases['direct_hubs_s'] = tick() - t
    t = tick()
    d.reassemble('lm_head', d.head_error(r.head))
    phases['head_s'] = tick() - t
    for kind, count in r.local.items():
        t = tick()
        for s_, e in d.local_errors(kind, count, targets).items():
            d.reassemble(s_, e)
        phases[f'local_{kind}_s'] = tick() - t
    t = tick()
    d.scalar_gradients(8)
    phases['scalars_s'] = tick() - t
    return dict(s_per_update=round(dt, 3), steps=steps, batch=8, seq_len=T_SEQ, loss=round(loss, 4),
                recipe='recipe(1.5) / 8 GPUs: writers 48, hidden 96, hubs 96, embedding 384, head 9216, '
                       'local q 72 v 72 gate 24 k 312 ve 864, nrep 16',
                reference_s_per_update_8xH100=10.38,
                phases={k: round(v, 3) for k, v in phases.items()})


def _lscpu():
    """The host's CPU description (lscpu) and how many CPUs this process may use."""
    import subprocess
    info = {}
    try:
        out = subprocess.run(['lscpu'], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(':')
            if key.strip() in ('Model name', 'CPU(s)', 'Thread(s) per core', 'Core(s) per socket', 'Socket(s)'):
                info[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    info['os.cpu_count'] = os.cpu_count()
    info['affinity'] = len(os.sched_getaffinity(0)) if hasattr(os, 'sched_getaffinity') else None
    return info


def _median_time(fn, reps):
    fn()  # warmup
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_baseline(model, sample_members=4, T=T_SEQ, reps=3):
    """The oracle (fp32 eager torch on the host cores) on bounded samples of the same workloads, 1 warmup then the
    median of `reps`: the population forward (the headline, in the metric's unit), config 1's GPT.forward and the
    eager config-3 credit readout (train/val/run.py:965-985, 1095-1101) at W = 2048 and 1024, each at torch's thread
    count on this host and at 1 thread (the reference harness's setting, train/val/run.py:2903)."""
    import torch
    from oracle import credit as oc
    from oracle import eggroll as oe
    from oracle import model as om
    ocfg = om.Config()
    threads = torch.get_num_threads()
    w = {n: p.detach().float().cpu() for n, p in model.named_parameters()}
    pairs = sample_members // 2
    offs = oe.step_offsets(ocfg, 0, 0, pairs)
    noise = oe.noise(ocfg, 0, offs, [j // 2 for j in range(sample_members)])
    sign = torch.tensor([0.002 if j % 2 == 0 else -0.002 for j in range(sample_members)])
    x, y = zipf_tokens(4, T, seed=0)
    g = torch.Generator().manual_seed(3)
    q = (torch.randn(16 * 8, T, 64, generator=g) / 8).bfloat16().float()
    k = (torch.randn(16 * 8, T, 64, generator=g) / 8).bfloat16().float()
    e = torch.randn(16 * 8, T, 64, generator=g)
    out = dict(kind='port', threads=threads, host=_lscpu())
    with torch.no_grad():
        med = _median_time(lambda: om.population_loss(w, ocfg, noise, sign, x[0], y[0]), reps)
        out.update(value=round(sample_members * T / med, 1), unit='member-tokens/s', cores=threads,
                   sample=f'{sample_members} members ({pairs} antithetic pairs) x 1 sequence x {T} tokens of the '
                   f'same population forward, oracle/model.py fp32 eager torch on {threads} threads; median of {reps} '
                   f'after 1 warmup ({med:.2f} s each)')
        c1, c3 = {}, {}
        for n_thr, rows_c1, rows_c3 in ((threads, 4, 128), (1, 1, 16)):
            torch.set_num_threads(n_thr)
            try:
                sec = _median_time(lambda: om.gpt_forward(w, ocfg, x[:rows_c1], y[:rows_c1], 'sum'), reps)
                c1[f'threads_{n_thr}'] = dict(rows=rows_c1, seconds=round(sec, 3),
                                              tokens_per_s=round(rows_c1 * T / sec, 1))
                for window in (T, 1024):
                    npairs = rows_c3 * sum(min(t, window) + 1 for t in range(T))
                    sec = _median_time(lambda: oc.credit_dense(q[:rows_c3], k[:rows_c3], e[:rows_c3], window), reps)
                    c3[f'threads_{n_thr}_window_{window}'] = dict(
                        rows=rows_c3, seconds=round(sec, 3), gflops=round(6 * 64 * npairs / sec / 1e9, 2))
            finally:
                torch.set_num_threads(threads)
    out['c1_gpt_forward'] = dict(c1, note='oracle gpt_forward, fp32 eager, [rows, 2048] Zipf(1.1) tokens, 8 layers; '
                                 'the 1-thread sample is 1 row')
    out['c3_eager_credit'] = dict(c3, note='oracle credit_dense = softmax(mask(q k^T / 8))^T @ e per (batch, head) '
                                  'row, T 2048; GFLOP/s at 6d per in-window pair; the 1-thread sample is 16 rows (2 '
                                  'batch entries x 8 heads) of the 128')
    return out


def peak_calibration(dev, iters=40000, workgroups=2048, reps=3, copy_bytes=4 << 30):
    """Measured ceilings on this box: the sustained bf16 MFMA rate (noise_peak_mfma: every CU, 8 independent
    v_mfma_f32_32x32x16_bf16 chains per wave, 2 waves per SIMD) on random N(0, 1) operands held in registers, on the
    same operands streamed from LDS every step (a GEMM main loop's fragment reads), and on zero operands (the clock
    depends on the operand bits); and the HBM rate of a plain device-to-device copy of 4 GiB (read + write bytes).
    Each figure is the best of `reps` launches timed with HIP events on the launch stream."""
    import torch
    from noise_amd import _lib
    n_rows = 4096
    g = torch.Generator(device=dev).manual_seed(17)
    rand = torch.randn(n_rows * 64 * 8, device=dev, generator=g).bfloat16()
    zero = torch.zeros_like(rand)
    out = torch.empty(workgroups * 256, device=dev)
    flop = workgroups * 4 * iters * 8 * 32768.0
    res = dict(unit='TFLOP/s', iters=iters, workgroups=workgroups, flop_per_launch=flop)
    stream = torch.cuda.current_stream(dev)
    for name, ops, lds in (('mfma_random_registers', rand, 0), ('mfma_random_lds', rand, 1),
                           ('mfma_zero_registers', zero, 0)):
        best = 0.0
        _lib.call('noise_peak_mfma', _lib.ptr(ops), n_rows, iters // 8, workgroups, lds, _lib.ptr(out),
                  _lib.stream(dev))  # warm-up (a shorter launch)
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            _lib.call('noise_peak_mfma', _lib.ptr(ops), n_rows, iters, workgroups, lds, _lib.ptr(out),
                      _lib.stream(dev))
            e1.record(stream)
            torch.cuda.synchronize()
            best = max(best, flop / (e0.elapsed_time(e1) * 1e-3) / 1e12)
        if not torch.isfinite(out).all():
            raise RuntimeError('peak calibration: non-finite accumulators')
        res[name] = round(best, 1)
        # the engine clock the rate implies, against the 2.5 PFLOP/s at 2.4 GHz of the spec sheet
        res[name + '_ghz'] = round(best / PEAK_BF16_TFLOPS * 2.4, 3)
    a = torch.ones(copy_bytes // 4, device=dev)
    b = torch.empty_like(a)
    b.copy_(a)
    best = 0.0
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        b.copy_(a)
        e1.record(stream)
        torch.cuda.synchronize()
        best = max(best, 2.0 * copy_bytes / (e0.elapsed_time(e1) * 1e-3) / 1e9)
    res['hbm_copy_gbs'] = round(best, 1)
    res['hbm_copy_bytes'] = copy_bytes
    del a, b
    res['note'] = ('mfma_*: TFLOP/s of a sustained v_mfma_f32_32x32x16_bf16 stream over every CU; _ghz: the clock '
                   'that rate implies (2.5 PFLOP/s at 2.4 GHz). hbm_copy_gbs: read + write bytes of one 4 GiB '
                   'device copy per second. The roofline\'s measured_peak is mfma_random_registers.')
    return res


def copy_calibration(dev, nbytes=1 << 30):
    """One device-to-device copy of `nbytes`: reads and writes exactly nbytes of HBM."""
    import torch
    a = torch.ones(nbytes // 4, device=dev)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps(dict(copy_calibration_bytes=nbytes)), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=10)
    ap.add_argument('--warmup', type=int, default=2)
    ap.add_argument('--workload', choices=['c4', 'c5'], default='c4')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--no-credit', action='store_true')
    ap.add_argument('--no-c2', action='store_true', help="skip config 2's single perturbed linear")
    ap.add_argument('--no-c5', action='store_true', help="skip config 5's full training step record")
    ap.add_argument('--no-dust', action='store_true', help="skip the head-slab estimator's line")
    ap.add_argument('--copy-calibration', action='store_true',
                    help='run one plain device copy of exactly 1 GiB and exit (rocprofv3 counter calibration)')
    ap.add_argument('--peak-calibration', action='store_true',
                    help='measure the sustained MFMA rate and the device-copy HBM rate on this box, print them, exit')
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) > 1:
        sys.exit('bench.py measures one GPU: this build runs the hot path on a single MI355X; '
                 'multi-GPU member sharding is design-only (see --gpus 1)')
    import torch
    from noise_amd import _lib
    _lib.lib()
    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        copy_calibration(dev)
        return
    if args.peak_calibration:
        print(json.dumps(dict(peak_calibration=peak_calibration(dev))), flush=True)
        return
    calib = peak_calibration(dev)
    res = bench_c4(args, dev) if args.workload == 'c4' else bench_c5(args, dev)
    model = res.pop('model')
    line = dict(metric=METRIC, value=round(res['value'], 1), unit='member-tokens/s', n_gpus=1, steps=args.steps,
                warmup=args.warmup, ms_per_step=round(res['ms_per_step'], 3), higher_is_better=True, scaling='weak',
                vs_baseline=None, dtype='bf16', data='synthetic (Zipf(1.1) tokens, random-init weights)',
                config=res['config'], roofline=res['roofline'])
    line['roofline']['forward_tflops'] = round(res['value'] * FLOP_PER_MEMBER_TOKEN / 1e12, 1)
    line['roofline']['forward_frac'] = round(res['value'] * FLOP_PER_MEMBER_TOKEN / 1e12 / PEAK_BF16_TFLOPS, 4)
    measured = calib['mfma_random_registers']
    line['roofline']['measured_peak'] = measured
    line['roofline']['frac_of_measured'] = round(line['roofline']['achieved'] / measured, 4)
    line['roofline']['forward_frac_of_measured'] = round(line['roofline']['forward_tflops'] / measured, 4)
    line['peak_calibration'] = calib
    line['kernels'] = res['kernels']
    line['finite'] = res['finite']
    if 'update' in res:
        line['update'] = res['update']
    if not args.no_credit:
        line['credit'] = bench_credit(dev)
    if not args.no_c2:
        line['c2'] = bench_c2(dev)
    if not args.no_c5 and args.workload == 'c4':
        line['c5'] = c5_record(dev)
    if args.workload == 'c4':
        line['c4_12layer'] = c4_12layer_record(dev)
        line['gpt_forward'] = bench_hooked_forward(dev, model)
    if not args.no_dust:
        line['dust_head_error'] = bench_head_error(dev)
        line['dust_direct'] = bench_dust_direct(dev, model)
        line['dust_step'] = bench_dust_step(dev)
    if not args.no_cpu_baseline:
        line['cpu_baseline'] = cpu_baseline(model)
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
