"""ctypes binding of libnoise_amd.so (include/noise_amd.h).

torch is imported first so that the HIP runtime torch ships (SONAME libamdhip64.so.7) is the one the library binds
to. There is no fallback: if the library is missing, every compute entry point raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (load order: torch's HIP runtime first)

LIB_PATH = Path(__file__).resolve().parent / 'libnoise_amd.so'
ABI_VERSION = 5  # include/noise_amd.h's signatures (noise_abi_version)
MAX_LAYERS = 16

c_p = ctypes.c_void_p
i32, i64, u64, f32, szt = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_size_t


class NoiseLayer(ctypes.Structure):
    _fields_ = [('w_qkv', c_p), ('w_proj', c_p), ('w_fc', c_p), ('w_mlp_proj', c_p), ('w_gate', c_p), ('ve', c_p),
                ('window', i32)]


class NoiseGpt(ctypes.Structure):
    _fields_ = [('n_layer', i32), ('vocab', i32), ('padded_vocab', i32), ('resid_lambdas', c_p), ('x0_lambdas', c_p),
                ('wte', c_p), ('lm_head', c_p), ('rope_cos', c_p), ('rope_sin', c_p),
                ('layers', NoiseLayer * MAX_LAYERS)]


class NoisePerturbation(ctypes.Structure):
    _fields_ = [('rows', c_p), ('stride', i64), ('n_rows', i64), ('resid_lambdas', i64), ('x0_lambdas', i64), ('wte', i64),
                ('lm_head', i64)] + [(n, i64 * MAX_LAYERS) for n in
                                     ('c_q', 'c_k', 'c_v', 'c_proj', 've_gate', 'c_fc', 'mlp_proj', 've')]


class NoiseDustDraws(ctypes.Structure):
    _fields_ = [('entry', i32), ('x_in', c_p), ('x0_in', c_p), ('sites', i32), ('sigma', f32), ('seed', u64),
                ('draw0', i32), ('n_draws', i32)]


_SIGNATURES = {
    'noise_last_error': ([], ctypes.c_char_p),
    'noise_abi_version': ([], ctypes.c_int),
    'noise_timing_enable': ([ctypes.c_int], ctypes.c_int),
    'noise_timing_read': ([i32, c_p, c_p, c_p], ctypes.c_int),
    'noise_peak_mfma': ([c_p, i64, i32, i32, i32, c_p, c_p], ctypes.c_int),
    'noise_rng_buffer': ([u64, u64, i64, c_p, c_p], ctypes.c_int),
    'noise_rng_offsets': ([u64, u64, c_p, i32, i64, c_p, c_p], ctypes.c_int),
    'noise_rng_rows': ([u64, c_p, i64, c_p, i32, c_p, i64, c_p, c_p], ctypes.c_int),
    'noise_lowrank': ([c_p, i32, c_p, c_p, i64, i64, i64, c_p, i64, i64, i64, i64, c_p, c_p, c_p, szt, c_p],
                      ctypes.c_int),
    'noise_lowrank_workspace': ([i64, i64, i64, i64, i32], szt),
    'noise_linear': ([c_p, i64, c_p, i64, i64, i64, c_p, i64, c_p], ctypes.c_int),
    'noise_lowrank_static': ([c_p, i32, c_p, c_p, i64, i64, i64, c_p, i64, i64, i64, i64, c_p, c_p, c_p], ctypes.c_int),
    'noise_attention': ([c_p, c_p, c_p, i64, i32, i64, i64, i64, i32, c_p, i64, i64, c_p, c_p], ctypes.c_int),
    'noise_population_forward_workspace': ([i64, i64], szt),
    'noise_population_forward': ([ctypes.POINTER(NoiseGpt), ctypes.POINTER(NoisePerturbation), c_p, c_p, i64, i64,
                                  c_p, c_p, c_p, i64, c_p, c_p, c_p, c_p, szt, c_p], ctypes.c_int),
    'noise_fitness': ([c_p, i64, i64, c_p, c_p, c_p], ctypes.c_int),
    'noise_outer_grad': ([c_p, i64, i64, i64, c_p, i64, i64, i64, f32, i32, c_p, c_p], ctypes.c_int),
    'noise_outer_grad_batch': ([c_p, i64, c_p, i64, ctypes.c_int32, c_p, c_p, c_p, c_p, c_p, f32, i32, c_p],
                               ctypes.c_int),
    'noise_reassemble': ([c_p, i64, c_p, i32, i64, i64, i64, i64, f32, c_p, c_p], ctypes.c_int),
    'noise_reassemble_embedding': ([c_p, i64, c_p, i64, i64, i64, c_p, c_p], ctypes.c_int),
    'noise_adamw': ([c_p, c_p, c_p, c_p, i64, f32, f32, f32, f32, f32, i64, c_p, c_p], ctypes.c_int),
    'noise_adamw_batch': ([i32, c_p, c_p, c_p, c_p, c_p, c_p, f32, f32, f32, f32, f32, i64, c_p], ctypes.c_int),
    'noise_credit_lse': ([c_p, c_p, i64, i64, i32, c_p, c_p], ctypes.c_int),
    'noise_credit_lse_bounded': ([c_p, c_p, i64, i64, i32, c_p, c_p], ctypes.c_int),
    'noise_lowrank_embed': ([c_p, i32, i64, i32, c_p, i64, c_p, i64, c_p, c_p, i32, i64, c_p, c_p], ctypes.c_int),
    'noise_credit_value': ([c_p, c_p, c_p, c_p, i64, i64, i32, i32, c_p, c_p], ctypes.c_int),
    'noise_credit_value_strided': ([c_p, c_p, c_p, c_p, i32, i64, i64, i64, i64, i32, i32, c_p, i32, i64, i64, c_p, c_p],
                                   ctypes.c_int),
    'noise_credit_key_context': ([c_p, c_p, c_p, c_p, i64, i64, i32, c_p, c_p, c_p], ctypes.c_int),
    'noise_head_error': ([c_p, i64, c_p, c_p, i32, i32, i32, i32, i32, f32, u64, c_p, c_p, szt, c_p], ctypes.c_int),
    'noise_head_error_workspace': ([i64, i32, i32], szt),
    'noise_dust_capture': ([ctypes.POINTER(NoiseGpt), c_p, c_p, i64, i64, c_p, c_p, c_p, szt, c_p], ctypes.c_int),
    'noise_dust_capture_sites': ([ctypes.POINTER(NoiseGpt), c_p, c_p, i64, i64, c_p, c_p, c_p, c_p, c_p, c_p, szt, c_p],
                                 ctypes.c_int),
    'noise_dust_rerun': ([ctypes.POINTER(NoiseGpt), ctypes.POINTER(NoiseDustDraws), c_p, c_p, i64, i64, c_p, c_p, szt,
                          c_p], ctypes.c_int),
    'noise_dust_workspace': ([i64, i64, i64], szt),
    'noise_dust_errors': ([c_p, c_p, i32, i64, i64, f32, f32, u64, i32, i32, i32, c_p, c_p, szt, c_p], ctypes.c_int),
    'noise_dust_errors_workspace': ([i32, i64, i64], szt),
    'noise_decayed_credit': ([c_p, i64, i64, i32, i32, f32, c_p, c_p], ctypes.c_int),
    'noise_dust_noise': ([u64, ctypes.c_uint32, ctypes.c_uint32, i32, i64, i32, c_p, c_p], ctypes.c_int),
    'noise_local_operand': ([i32, u64, ctypes.c_uint32, ctypes.c_uint32, i32, i32, i32, c_p, c_p, c_p, c_p, c_p, f32, c_p, c_p],
                            ctypes.c_int),
    'noise_local_score': ([c_p, c_p, c_p, i32, i32, i32, c_p, c_p], ctypes.c_int),
    'noise_local_estimate': ([c_p, u64, ctypes.c_uint32, ctypes.c_uint32, i32, i32, i32, i32, f32, c_p, c_p], ctypes.c_int),
    'noise_attention_periodic': ([c_p, i32, c_p, i32, c_p, i32, i64, i32, i64, i64, i64, i32, i32, c_p, i64, i64, c_p],
                                 ctypes.c_int),
}

EXPORTS = tuple(_SIGNATURES)

_lib = None


def lib():
    """The loaded library; raises if it was never built (no CPU fallback exists)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f'{LIB_PATH} is missing: build it with `python -m noise_amd.build`')
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        if handle.noise_abi_version() != ABI_VERSION:
            raise RuntimeError(f'{LIB_PATH} has ABI version {handle.noise_abi_version()}, these bindings expect '
                               f'{ABI_VERSION}: rebuild it with `python -m noise_amd.build`')
        _lib = handle
    return _lib


def check(rc):
    """Turn a NOISE_ERR_* code into the Python exception the reference's ops raise for the same failure."""
    if rc == 0:
        return
    msg = lib().noise_last_error().decode(errors='replace')
    if rc in (1, 3):
        raise ValueError(msg)
    raise RuntimeError(msg)


def call(name, *args):
    check(getattr(lib(), name)(*args))


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_device(*tensors):
    for t in tensors:
        if t is not None and t.device.type != 'cuda':
            raise ValueError(f'noise_amd kernels take device tensors, got a tensor on {t.device}')


def timing_enable(on=True):
    lib().noise_timing_enable(int(on))


def timing_read():
    """class name -> (launch count, total milliseconds) of the launches timed since timing_enable()."""
    n = 32
    counts = (ctypes.c_int64 * n)()
    ms = (ctypes.c_double * n)()
    names = (ctypes.c_char_p * n)()
    k = lib().noise_timing_read(n, counts, ms, names)
    return {names[c].decode(): (counts[c], ms[c]) for c in range(min(k, n))}
