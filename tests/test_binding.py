"""The executor binding: only the hot-path attributes of the executor's
kernels module change (damendaemon/qwen2.py:458-461 holds the module; the
executor also calls swiglu at paged.py:114, rope_store at qwen2.py:606,
linear_fp32 at qwen2.py:678 and rms at qwen2.py:684)."""
import types

import pytest

import damendaemon_amd.kernels as amd


def _reference_like():
    mod = types.ModuleType('damendaemon.kernels')
    for name in ('rms', 'swiglu', 'rope_store', 'linear_fp32', 'attention', 'rope_batch', 'copy_pages'):
        setattr(mod, name, (lambda n: (lambda *a, **k: n))(name))
    return mod


def test_install_replaces_only_the_hot_path():
    mod = _reference_like()
    before = dict(vars(mod))
    assert amd.install(mod) is mod
    assert mod.attention is amd.attention and mod.rope_batch is amd.rope_batch
    for name in ('rms', 'swiglu', 'rope_store', 'linear_fp32', 'copy_pages'):
        assert getattr(mod, name) is before[name]
        assert getattr(mod, name)() == name
    assert set(vars(mod)) == set(before)


def test_overlay_leaves_the_module_alone():
    mod = _reference_like()
    before = dict(vars(mod))
    view = amd.overlay(mod)
    assert dict(vars(mod)) == before
    assert view.attention is amd.attention and view.rope_batch is amd.rope_batch
    for name in ('rms', 'swiglu', 'rope_store', 'linear_fp32'):
        assert getattr(view, name) is before[name]


def test_executor_style_calls_resolve():
    """The attribute lookups the paged executor makes all resolve after binding."""
    executor = types.SimpleNamespace(kernels=_reference_like())
    amd.install(executor.kernels)
    assert executor.kernels.swiglu() == 'swiglu'
    assert executor.kernels.rms() == 'rms'
    assert executor.kernels.rope_store() == 'rope_store'
    assert executor.kernels.linear_fp32() == 'linear_fp32'
    assert executor.kernels.attention is amd.attention


def test_install_rejects_a_non_kernels_module():
    with pytest.raises(ValueError):
        amd.install(types.ModuleType('empty'))
