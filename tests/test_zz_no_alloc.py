"""The allocation-free decode entry point (dd_decode_attention_static)
against dd_decode_attention on the same inputs, through the C ABI.

Both run the same split and merge kernels; only where the split partials
live differs (a static device array instead of caller buffers), so the
outputs must agree bit for bit.  Two calls in a row, the second smaller,
check that leftovers of the first call in the shared array do not leak into
the second.
"""
import ctypes

import pytest
import torch

from damendaemon_amd import _native, kernels
from damendaemon_amd.workloads import paged_decode_case

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def static_call(launch, out):
    """The launch's dd_decode_attention arguments, minus partial/lse, into `out`."""
    args = list(launch._args)
    args = args[:-5] + [_native.ptr(out)] + args[-2:]
    stream = ctypes.c_void_p(torch.cuda.current_stream(out.device).cuda_stream)
    _native.call('dd_decode_attention_static', *args, stream)


def case_on_device(contexts, heads, kvh, dim, dtype, seed):
    case = paged_decode_case(contexts, heads, kvh, dim, dtype, seed=seed, nan_fill=True)
    return {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}


def run_both(case, **kw):
    launch = kernels.prepare_attention(case['query'], case['cache_k'], case['cache_v'], case['positions'],
                                       case['slots'], page_table=case['page_table'], **kw)
    assert launch.splits > 1, 'the case must exercise the split scratch'
    ref = launch.run().clone()
    out = torch.full_like(ref, float('nan'))
    static_call(launch, out)
    torch.cuda.synchronize()
    return ref, out


def test_static_matches_allocating_entry_two_calls():
    big = case_on_device([9000, 300, 4097, 7000, 64, 12000], 32, 8, 128, torch.bfloat16, seed=1)
    small = case_on_device([2500, 17], 8, 2, 128, torch.bfloat16, seed=2)
    for case in (big, small):
        ref, out = run_both(case)
        assert torch.equal(out, ref)


def test_static_int8_and_sinks():
    case = paged_decode_case([5000, 900, 3333], 16, 4, 128, torch.float32, seed=3)
    from oracle import paged_oracle as O
    qk, ks = O.quantize_q8(case['cache_k'], 128)
    qv, vs = O.quantize_q8(case['cache_v'], 128)
    case.update(cache_k=qk, cache_v=qv, query=case['query'].to(torch.bfloat16))
    dev = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    sinks = torch.randn(16, generator=torch.Generator().manual_seed(4)).to(DEV)
    ref, out = run_both(dev, k_scale=ks.to(DEV), v_scale=vs.to(DEV), sinks=sinks)
    assert torch.equal(out, ref)


def test_static_rejects_oversized_batch():
    case = case_on_device([40000], 32, 8, 128, torch.bfloat16, seed=5)
    launch = kernels.prepare_attention(case['query'], case['cache_k'], case['cache_v'], case['positions'],
                                       case['slots'], page_table=case['page_table'])
    args = list(launch._args)
    args[13] = 70000   # batch far beyond the static array (rows are never read: the call is refused first)
    args = args[:-5] + [_native.ptr(launch.out)] + args[-2:]
    lib = _native.library()
    code = lib.dd_decode_attention_static(*args, ctypes.c_void_p(0))
    assert code == 4  # DD_ESCRATCH
