"""The C-ABI library loads on a CPU-only host and exports every symbol the header declares."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / 'include' / 'damendaemon_amd.h'


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(dd_[a-z0-9_]+)\s*\(', text)))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert 'dd_abi_version' in names and 'dd_decode_attention' in names


def test_library_exports_every_declared_symbol():
    from damendaemon_amd import _native
    if not _native.LIBRARY.exists():
        pytest.fail('library not built: run python -m damendaemon_amd.build')
    lib = ctypes.CDLL(str(_native.LIBRARY))
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_abi_version_and_python_signatures():
    from damendaemon_amd import _native
    lib = _native.library()
    assert lib.dd_abi_version() == _native.ABI_VERSION
    assert set(_native.SIGNATURES) <= set(declared_symbols())
    assert lib.dd_error_string(1) == b'invalid argument'


def test_split_policy_covers_context():
    from damendaemon_amd import _native
    lib = _native.library()
    for ctx, bkh in [(1024, 8), (8192, 512), (32768, 32), (16, 1), (513, 3)]:
        tokens = ctypes.c_int()
        splits = lib.dd_decode_splits(ctx, bkh, ctypes.byref(tokens))
        assert splits >= 1 and tokens.value % 64 == 0
        assert splits * tokens.value >= ctx > (splits - 1) * tokens.value
    assert lib.dd_decode_splits(0, 1, None) < 0


def test_split_policy_for_head_size():
    """The head-size-aware policy equals the plain one except for int8 pages
    (longer splits) and at head sizes 160-256 with 16-bit pages, many
    (sequence, KV head) pairs and few splits per resident workgroup, where
    splits hold at most 768 keys."""
    from damendaemon_amd import _native
    lib = _native.library()

    def policy(ctx, bkh, dim, dtype):
        tokens = ctypes.c_int()
        splits = lib.dd_decode_splits_for(ctx, bkh, dim, dtype, ctypes.byref(tokens))
        return splits, tokens.value

    def plain(ctx, bkh):
        tokens = ctypes.c_int()
        splits = lib.dd_decode_splits(ctx, bkh, ctypes.byref(tokens))
        return splits, tokens.value

    assert policy(8192, 256, 256, _native.BF16) == (11, 768)     # 64 sequences x 4 KV heads
    assert policy(8192, 256, 160, _native.F16) == (11, 768)
    assert policy(8192, 256, 128, _native.BF16) == plain(8192, 256)
    assert policy(8192, 512, 256, _native.BF16) == (6, 1408)     # 8 KV heads: six splits each, enough units
    assert policy(32768, 32, 256, _native.BF16) == (16, 2048)    # C5
    assert policy(8192, 512, 128, _native.BF16) == (6, 1408)     # C2
    assert policy(8192, 512, 128, _native.I8) == (3, 2752)       # C3: longer int8 splits
    assert policy(32768, 32, 256, _native.I8) == (16, 2048)      # the 512-workgroup floor wins
    for ctx in (300, 1000, 4096, 8192, 32768):
        for bkh in (1, 8, 100, 128, 300, 512, 4096):
            for dim, dtype in ((64, _native.BF16), (128, _native.F32), (256, _native.F32)):
                assert policy(ctx, bkh, dim, dtype) == plain(ctx, bkh)
            splits, st = policy(ctx, bkh, 128, _native.I8)
            assert st % 64 == 0 and plain(ctx, bkh)[1] <= st <= max(2752, plain(ctx, bkh)[1])
            assert splits * st >= ctx > (splits - 1) * st
            assert st == plain(ctx, bkh)[1] or bkh * splits >= 512
            splits, st = policy(ctx, bkh, 224, _native.BF16)
            assert st % 64 == 0 and 256 <= st <= plain(ctx, bkh)[1]
            assert splits * st >= ctx > (splits - 1) * st
    assert lib.dd_decode_splits_for(0, 1, 256, _native.BF16, None) < 0


def test_split_policy_sizes_and_occupancy():
    """Split sizes are multiples of 64 in [256, 2048]; the tuned configurations keep
    theirs (64 x 8 KV heads over 8192-key tables: 1408; 16 x 2 over 32768: 2048); and
    a launch has about 512 workgroups or more unless the 256-key floor stops it."""
    from damendaemon_amd import _native
    lib = _native.library()

    def policy(ctx, bkh):
        tokens = ctypes.c_int()
        splits = lib.dd_decode_splits(ctx, bkh, ctypes.byref(tokens))
        return splits, tokens.value

    assert policy(8192, 512) == (6, 1408)
    assert policy(32768, 32) == (16, 2048)
    for ctx in (300, 1000, 4096, 8192, 32768, 131072):
        for bkh in (1, 8, 64, 100, 512, 4096):
            splits, st = policy(ctx, bkh)
            assert st % 64 == 0 and 256 <= st <= 2048
            assert splits * st >= ctx > (splits - 1) * st
            # rounding split sizes up to 64 keys may cost one split
            assert splits * bkh >= 0.8 * 512 or st == 256, (ctx, bkh, splits, st)
