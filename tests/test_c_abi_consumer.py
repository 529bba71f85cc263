"""The library's host-side entry points are callable from plain C through the
header alone (the binding a cgo / JNI / N-API host would write); CPU only."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_plain_c_caller(tmp_path):
    from damendaemon_amd import _native
    if not _native.LIBRARY.exists():
        pytest.fail('library not built: run python -m damendaemon_amd.build')
    cc = shutil.which('gcc') or shutil.which('cc')
    if cc is None:
        pytest.skip('no C compiler on this host')
    exe = tmp_path / 'abi_consumer'
    lib_dir = _native.LIBRARY.parent
    subprocess.run([cc, '-std=c99', '-O1', '-Wall', '-Werror', str(ROOT / 'tests' / 'c' / 'abi_consumer.c'),
                    '-I', str(ROOT / 'include'), '-L', str(lib_dir), '-ldamendaemon_amd',
                    f'-Wl,-rpath,{lib_dir}', '-o', str(exe)], check=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stderr
    assert run.stdout.startswith('ok:')
