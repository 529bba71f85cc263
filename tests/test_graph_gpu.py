"""Decode attention captured in a HIP graph (the reference captures its decode
step, damendaemon/batch.py:25-46): every replay must reproduce the eager
result bit for bit, with eager work and synchronisations between replays."""
import pytest
import torch

from damendaemon_amd import kernels
from damendaemon_amd.workloads import paged_decode_case

pytestmark = pytest.mark.gpu
DEV = 'cuda'


@pytest.mark.parametrize('kind', ['bf16', 'int8'])
def test_decode_graph_replays_match_eager(kind):
    case = paged_decode_case([17, 600, 2500, 4097, 9000], 32, 8, 128, torch.bfloat16, seed=31)
    d = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    ks = vs = None
    if kind == 'int8':
        from damendaemon_amd import kv_quant
        ck, ks = kv_quant.quantize_kv(d['cache_k'], group=128)
        cv, vs = kv_quant.quantize_kv(d['cache_v'], group=128)
        d['cache_k'], d['cache_v'] = ck, cv
    launch = kernels.prepare_attention(d['query'], d['cache_k'], d['cache_v'], d['positions'], d['slots'],
                                       page_table=d['page_table'], k_scale=ks, v_scale=vs)
    assert launch.splits > 1
    eager = launch.run().clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch.run()
    for i in range(3):
        launch.out.fill_(float('nan'))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(launch.out, eager), f'replay {i} differs from the eager launch'
        torch.randn(1024, device=DEV).sum().item()  # unrelated eager work between replays


@pytest.mark.filterwarnings('ignore:The CUDA Graph is empty')
@pytest.mark.parametrize('dim', [128, 256])
def test_prefill_graph_replays_match_eager(dim):
    """A prepared prefill launch (plan uploaded, flags allocated) captured in a
    HIP graph: its persistent schedule and re-run flags replay exactly.  The
    host-side preparation itself cannot be captured (it uploads through reused
    pinned buffers) and says so."""
    from damendaemon_amd import packing, ragged
    lengths, starts = [1, 70, 300, 129], [0, 40, 900, 2000]
    contexts = [s + n for s, n in zip(starts, lengths)]
    case = paged_decode_case(contexts, 16, 4, dim, torch.bfloat16, seed=dim)
    d = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    q = torch.randn(sum(lengths), 16, dim, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(DEV)
    packed = packing.pack_batch(lengths, starts, list(range(len(lengths))), d['page_table'])
    launch = ragged.prepare_prefill(q, d['cache_k'], d['cache_v'], packed, d['page_table'])
    eager = launch.run().clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch.run()
    for i in range(3):
        launch.out.fill_(float('nan'))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(launch.out, eager), f'replay {i} differs from the eager launch'
        torch.randn(1024, device=DEV).sum().item()
    with pytest.raises(RuntimeError, match='graph capture'):
        with torch.cuda.graph(torch.cuda.CUDAGraph()):
            ragged.prepare_prefill(q, d['cache_k'], d['cache_v'], packed, d['page_table'])
