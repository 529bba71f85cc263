"""Compile the gfx950 HIP sources under csrc/ into one shared library.

Objects are built in parallel with hipcc and linked into
``damendaemon_amd/_lib/libdamendaemon_amd.so`` (in-tree, so the library
travels with the source tree).  Every call recompiles: the build is the
"does it build" check as well as the way to refresh the library.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / 'csrc'
OUT_DIR = HERE / '_lib'
LIBRARY = OUT_DIR / 'libdamendaemon_amd.so'
ARCH = 'gfx950'
HIPCC = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')
FLAGS = ['-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}',
         # Packed FP32 instructions are kept out of every kernel.
         '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
         '-Wno-unused-command-line-argument']


# Per-source extra flags.  The streamed decode kernels keep their MFMA
# accumulators in VGPRs: in the AGPR form the compiler copies them between
# the two register files on every loop iteration.
_VGPR_MFMA = ['-mllvm', '-amdgpu-mfma-vgpr-form=1']
SOURCE_FLAGS = {'decode_bf16.hip': _VGPR_MFMA, 'decode_f16.hip': _VGPR_MFMA, 'decode_i8.hip': _VGPR_MFMA}


def _compile(source, obj, extra=()):
    cmd = [HIPCC, *FLAGS, *SOURCE_FLAGS.get(source.name, []), *extra, '-c', str(source), '-o', str(obj)]
    run = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = '\n'.join(l for l in run.stderr.splitlines() if noise not in l)
    if run.returncode:
        raise RuntimeError(f'hipcc failed for {source.name}:\n{err}')
    return err


def build(jobs=None, verbose=False, extra_flags=(), library=LIBRARY):
    """Compile and link; ``extra_flags`` (e.g. -D tuning macros) and
    ``library`` allow side-by-side variant builds."""
    library = Path(library)
    OUT_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob('*.hip'))
    tag = library.stem
    objs = [OUT_DIR / f'{s.stem}.{tag}.o' for s in sources]
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)), 16)
    with ThreadPoolExecutor(jobs) as pool:
        for warn in pool.map(lambda s, o: _compile(s, o, extra_flags), sources, objs):
            if warn and verbose:
                print(warn, file=sys.stderr)
    tmp = library.with_suffix('.so.tmp')
    link = [HIPCC, '-shared', f'--offload-arch={ARCH}', *map(str, objs), '-o', str(tmp)]
    run = subprocess.run(link, capture_output=True, text=True)
    if run.returncode:
        raise RuntimeError('link failed:\n' + run.stderr)
    os.replace(tmp, library)
    for o in objs:
        o.unlink()
    return library


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv))
