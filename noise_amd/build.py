"""Build libnoise_amd.so, the HIP (gfx950) library behind noise_amd, in-tree with hipcc.

    python -m noise_amd.build          # or __graft_entry__.build()
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / 'csrc'
OUT = HERE / 'libnoise_amd.so'
OBJ = HERE / '_build'
ARCH = os.environ.get('NOISE_AMD_ARCH', 'gfx950')

HIP_FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-Wall', '-Wno-unused-function',
    '-fhip-fp32-correctly-rounded-divide-sqrt',
    # packed fp32 VALU ops stay off (hipcc's host pass does not know the feature and warns; harmless)
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
]


def hipcc():
    path = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not Path(path).exists():
        raise RuntimeError('hipcc not found: the HIP library cannot be built')
    return path


def _compile(src: Path) -> Path:
    obj = OBJ / (src.name + '.o')
    cmd = [hipcc(), *HIP_FLAGS, '-c', str(src), '-o', str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = [l for l in res.stderr.splitlines() if 'packed-fp32-ops' not in l]
    if res.returncode != 0:
        raise RuntimeError(f'hipcc failed on {src.name}:\n' + '\n'.join(noise))
    if noise:
        print('\n'.join(noise), file=sys.stderr)
    return obj


def build(verbose=True) -> Path:
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob('*.hip')) + sorted(CSRC.glob('*.cpp'))
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = OUT.with_suffix('.so.tmp')
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', *map(str, objs), '-o', str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError('link failed:\n' + res.stderr)
    os.replace(tmp, OUT)
    if verbose:
        print(f'built {OUT} from {len(sources)} sources')
    return OUT


if __name__ == '__main__':
    build()
