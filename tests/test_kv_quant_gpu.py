"""GPU Q8_0 codec: bit-exact against the CPU oracle (kv_quant.py:48-76 arithmetic)."""
import pytest
import torch

from damendaemon_amd import kv_quant
from oracle import paged_oracle as oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize('dim,group', [(128, 32), (128, 128), (96, 32), (64, 64), (80, 16), (256, 32)])
def test_quantize_bit_exact(dtype, dim, group):
    g = torch.Generator().manual_seed(dim + group)
    x = (torch.randn(3, 5, 37, dim, generator=g) * torch.rand(3, 5, 37, 1, generator=g) * 4).to(dtype)
    x[0, 0, 0] = 0                                  # all-zero groups
    x[0, 0, 1, :group] = torch.linspace(-1, 1, group).to(dtype)
    q, s = kv_quant.quantize_kv(x.cuda(), group)
    eq, es = oracle.quantize_q8(x, group)
    assert torch.equal(q.cpu(), eq)
    assert torch.equal(s.cpu().view(torch.int16), es.view(torch.int16))
    back = kv_quant.dequantize_kv(q, s, torch.float32).cpu()
    assert torch.equal(back, oracle.dequantize_q8(eq, es))


def test_reference_default_group():
    x = torch.randn(2, 4, 9, 128).cuda()
    q, s = kv_quant.quantize_kv(x)
    assert s.shape == (2, 4, 9, 4)
    eq, es = oracle.quantize_q8(x.cpu(), 32)
    assert torch.equal(q.cpu(), eq) and torch.equal(s.cpu(), es)


def test_store_and_read_dense_slots():
    data, scales = kv_quant.allocate_kv(3, 2, 40, 64, 'cuda')
    k = torch.randn(2, 2, 5, 64).cuda()
    v = torch.randn(2, 2, 5, 64).cuda()
    slots = torch.tensor([2, 0]).cuda()
    pos = torch.tensor([[0, 1, 2, 3, 4], [10, 11, 12, 13, 14]]).cuda()
    kv_quant.store_kv((data, scales), slots, pos, k, v)
    rk, rv = kv_quant.read_kv((data, scales), torch.tensor([2]).cuda(), 5)
    eq, es = oracle.quantize_q8(k[0].cpu(), 32)
    assert torch.equal(rk[0].cpu(), oracle.dequantize_q8(eq, es))


def test_store_duplicate_rows_last_wins():
    """Two rows writing the same (slot, position): the later row's values
    stay, as in the reference's row-by-row loop (kv_quant.py:99-106)."""
    data, scales = kv_quant.allocate_kv(2, 2, 16, 64, 'cuda')
    g = torch.Generator().manual_seed(5)
    k = torch.randn(3, 2, 4, 64, generator=g).cuda()
    v = torch.randn(3, 2, 4, 64, generator=g).cuda()
    slots = torch.tensor([1, 0, 1]).cuda()
    pos = torch.tensor([[0, 1, 2, 3], [0, 1, 2, 3], [2, 3, 4, 3]]).cuda()
    kv_quant.store_kv((data, scales), slots, pos, k, v)
    rk, rv = kv_quant.read_kv((data, scales), torch.tensor([1]).cuda(), 5)
    # slot 1: positions 0, 1 from row 0; 2 from row 2 (token 0); 3 from row 2's
    # last token (token 3, which also beats its own token 1); 4 from row 2
    want_k = torch.stack([k[0, :, 0], k[0, :, 1], k[2, :, 0], k[2, :, 3], k[2, :, 2]], dim=1).cpu()
    want_v = torch.stack([v[0, :, 0], v[0, :, 1], v[2, :, 0], v[2, :, 3], v[2, :, 2]], dim=1).cpu()
    eq, es = oracle.quantize_q8(want_k, 32)
    assert torch.equal(rk[0].cpu(), oracle.dequantize_q8(eq, es))
    eq, es = oracle.quantize_q8(want_v, 32)
    assert torch.equal(rv[0].cpu(), oracle.dequantize_q8(eq, es))
