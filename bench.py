"""Benchmark of the paged decode attention hot path on one MI355X.

One step = one ragged paged decode attention over the whole batch
(BASELINE config C2 by default: 64 sequences, contexts U[512, 8192] seeded,
32 query / 8 KV heads, head_dim 128, bf16 pages of 16 tokens scattered over
a pool 1.25x the pages used), inputs resident in HBM before timing.

Prints ONE JSON line (the driver's contract) with:
  value        tokens/s = sequences per step / wall time per step, the steps
               (split kernel + merge) launched back to back on the stream;
               the same step replayed alone from a HIP graph is reported as
               config.graph_replay_ms_per_step
  roofline     the split kernel (dominant) timed with HIP events on its own
               stream: algorithmic bytes per launch / its mean duration,
               against MI355X's 8 TB/s HBM3E peak
  cpu_baseline the PyTorch CPU restatement (page gather + masked GQA SDPA,
               fp32) timed on the whole batch with every core of the
               affinity mask (a few seconds per step)
  other_configs  (a run without --config only) C3, C4 and C5 measured in the same run:
               value, ms_per_step and roofline of each (their own lines via
               --config)
Extra configurations (--config c2f32 / c3 / c3g32 / c4 / c4f32 / c5 / c5f32 / rope / copy) print
their own lines; the default line is C2.
"""
import argparse
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBPS = 8000.0   # MI355X HBM3E, AMD datasheet
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, AMD datasheet
PEAK_FP32_TFLOPS = 157.3   # MI355X dense fp32 MFMA, AMD datasheet


def algorithmic_bytes(case, kv_bytes_per_token_head):
    """KV bytes read + Q read + O written + page-table entries read, one step."""
    B, H, _, D = case['query'].shape
    KH = case['cache_k'].shape[1]
    ctx = sum(case['contexts'])
    pages = sum(-(-c // 16) for c in case['contexts'])
    q_o = 2 * B * H * D * case['query'].element_size()
    return ctx * KH * kv_bytes_per_token_head + q_o + pages * 4


# Kernel families and the sources each one is compiled from (besides common.h
# and the public header): a profile summary records the digest of its family.
DIGEST_FAMILIES = {
    'decode': ('decode', 'q8.h'),
    'prefill': ('prefill',),
    'rope': ('rope',),
    'copy': ('copy',),
}


def source_digest(family=None):
    """sha256 over the HIP sources of one kernel family (csrc/ files whose name
    starts with one of its prefixes, plus common.h and the public header), or
    over every source when family is None: ties a profile summary to the
    kernels it measured."""
    import hashlib
    csrc = os.path.join(ROOT, 'damendaemon_amd', 'csrc')
    prefixes = DIGEST_FAMILIES[family] if family else ('',)
    h = hashlib.sha256()
    files = [os.path.join(csrc, n) for n in sorted(os.listdir(csrc))
             if n.endswith(('.hip', '.h')) and (n == 'common.h' or n.startswith(prefixes))]
    files.append(os.path.join(ROOT, 'include', 'damendaemon_amd.h'))
    for path in files:
        h.update(os.path.basename(path).encode())
        with open(path, 'rb') as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(summary, family='decode'):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    PMC summary profiles/<summary>.md (FETCH_SIZE + WRITE_SIZE, calibrated
    against a plain copy), or None when there is none or it was taken on
    other kernel sources than the ones running now."""
    path = os.path.join(ROOT, 'profiles', f'{summary}.md')
    if not os.path.exists(path):
        return None
    fields = {}
    for line in open(path):
        if ':' in line and not line.startswith(('#', '|', ' ')):
            key, _, val = line.partition(':')
            fields[key.strip()] = val.strip().strip('`')
    if fields.get('source_digest') != source_digest(family) or 'traffic_bytes_per_launch' not in fields:
        return None
    return int(fields['traffic_bytes_per_launch'])


def cpu_baseline_mixed(case, n_chunks, budget_s=20.0):
    """The mixed batch's attention on the host cores the way the reference's
    executor runs it there: per prefill chunk a page gather and a lower-right
    causal SDPA (oracle.prefill_attention_sdpa), and the decode rows through
    oracle.decode_attention_sdpa, fp32, every core of this process."""
    from oracle import paged_oracle
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    lengths, starts, slots = case['lengths'], case['starts'], case['seg_slots']
    table, ck, cv, q = (case[k].cpu() for k in ('page_table', 'cache_k', 'cache_v', 'q'))
    t_pre = sum(lengths[:n_chunks])
    dec_pos = torch.tensor(starts[n_chunks:], dtype=torch.int64)
    dec_slots = torch.tensor(slots[n_chunks:], dtype=torch.int64)

    def step():
        paged_oracle.prefill_attention_sdpa(q[:t_pre], ck, cv, lengths[:n_chunks], starts[:n_chunks],
                                            slots[:n_chunks], table)
        paged_oracle.decode_attention_sdpa(q[t_pre:].unsqueeze(2), ck, cv, dec_pos, dec_slots, table)

    step()   # warm-up
    times = []
    start = time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - start < budget_s and len(times) < 5):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {'value': sum(lengths) / med, 'unit': 'tokens/s', 'cores': threads, 'kind': 'port',
            'sample': f'the whole batch ({n_chunks} chunks of {lengths[0]} tokens + {len(lengths) - n_chunks} '
                      f'decode rows): fp32 page gather + SDPA per chunk and for the decode rows on {threads} '
                      f'threads, median of {len(times)} steps'}


def build_case(name, device):
    from damendaemon_amd import workloads, kv_quant
    if name == 'c2':
        case = workloads.config_c2(device=device)
        D = case['query'].shape[-1]
        return case, 'C2 ragged paged decode bf16: 64 seqs, ctx U[512,8192] seed 2, H32/KH8/D128, page 16', \
            'bf16', algorithmic_bytes(case, 2 * D * 2)
    if name == 'c3':
        case = workloads.config_c2(device=device)
        D = case['query'].shape[-1]
        case = workloads.quantize_pages(case, D, kv_quant)
        return case, 'C3 ragged paged decode int8 KV (fp16 scale per token-head): C2 shapes', 'int8', \
            algorithmic_bytes(case, 2 * (D + 2))
    if name == 'c2f32':
        import torch
        case = workloads.config_c2(device=device, dtype=torch.float32)
        D = case['query'].shape[-1]
        return case, 'C2 shapes with fp32 pages (a float32 compute dtype): 64 seqs, ctx U[512,8192] seed 2, H32/KH8/D128', \
            'f32', algorithmic_bytes(case, 2 * D * 4)
    if name == 'c3g32':
        case = workloads.config_c2(device=device)
        D = case['query'].shape[-1]
        case = workloads.quantize_pages(case, 32, kv_quant)
        return case, 'C3 ragged paged decode int8 KV, reference group-32 scales (fp16 per 32 channels): C2 shapes', \
            'int8', algorithmic_bytes(case, 2 * (D + 2 * (D // 32)))
    if name == 'c5f32':
        import torch
        case = workloads.paged_decode_case([32768] * 16, 16, 2, 256, torch.float32, seed=5, device=device,
                                           capacity=16 * 2048, outlier_frac=0.01)
        D = case['query'].shape[-1]
        return case, 'C5 shapes with fp32 pages: 16 x 32768, H16/KH2/D256, 1% K outliers x8', 'f32', \
            algorithmic_bytes(case, 2 * D * 4)
    if name == 'c5':
        case = workloads.config_c5(device=device)
        D = case['query'].shape[-1]
        return case, 'C5 long split-KV decode bf16: 16 x 32768, H16/KH2/D256, 1% K outliers x8', 'bf16', \
            algorithmic_bytes(case, 2 * D * 2)
    raise SystemExit(f'unknown config {name}')


def cpu_baseline(case, budget_s=20.0):
    """Time oracle.decode_attention_sdpa (fp32, CPU) on the whole batch, with
    every core of this process's affinity mask."""
    from oracle import paged_oracle
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    n = case['query'].shape[0]
    table = case['page_table']
    used = torch.unique(table[table >= 0]).long()
    remap = torch.full((case['cache_k'].shape[0],), -1, dtype=torch.int64, device=used.device)
    remap[used] = torch.arange(used.numel(), device=used.device)
    small_table = torch.where(table >= 0, remap[table.clamp_min(0).long()], -1).to(torch.int32).cpu()
    k = case['cache_k'][used].cpu()
    v = case['cache_v'][used].cpu()
    q = case['query'].cpu()
    pos = case['positions'].cpu()
    slots = torch.arange(n)
    if k.dtype == torch.int8:
        k = paged_oracle.dequantize_q8(k, case['k_scale'][used].cpu())
        v = paged_oracle.dequantize_q8(v, case['v_scale'][used].cpu())
    paged_oracle.decode_attention_sdpa(q, k, v, pos, slots, small_table)   # warm-up
    times = []
    start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - start < budget_s and len(times) < 10):
        t0 = time.perf_counter()
        paged_oracle.decode_attention_sdpa(q, k, v, pos, slots, small_table)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {'value': n / med, 'unit': 'tokens/s', 'cores': threads, 'kind': 'port',
            'sample': f'all {n} sequences (ctx sum {sum(case["contexts"])}), fp32 page gather + masked GQA '
                      f'SDPA on {threads} threads, median of {len(times)} steps'}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=50)
    ap.add_argument('--warmup', type=int, default=5)
    ap.add_argument('--ragged', action='store_true',
                    help='c4/c4f32: also time ragged_attention (decode rows overlapped on a side stream)')
    ap.add_argument('--config', default='c2', choices=['c2', 'c2f32', 'c3', 'c3g32', 'c4', 'c4f32', 'c5', 'c5f32', 'rope', 'copy'])
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--no-other-configs', action='store_true',
                    help='c2: leave out the C3 / C4 / C5 summaries of the default line')
    ap.add_argument('--head-dim', type=int, default=128,
                    help='c4/c4f32: head size of the mixed batch (BASELINE C4 is 128)')
    ap.add_argument('--copy-probe', action='store_true',
                    help='only run 1 GiB device-to-device copies (calibrates rocprofv3 FETCH/WRITE_SIZE)')
    args = ap.parse_args()
    if args.copy_probe:
        src = torch.randn(1 << 28, device='cuda:0')      # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({'copy_probe_bytes_each_way': src.numel() * 4, 'copies': 5}))
        return
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one GPU only: this build has no multi-GPU path '
              '(decode shards by sequence with no exchange; see the design notes)', file=sys.stderr)
        raise SystemExit(2)

    dev = 'cuda:0'
    torch.cuda.set_device(0)
    if args.config == 'c4':
        line = bench_mixed(args, dev)
    elif args.config == 'c4f32':
        line = bench_mixed(args, dev, torch.float32)
    elif args.config == 'rope':
        line = bench_rope(args, dev)
    elif args.config == 'copy':
        line = bench_copy(args, dev)
    else:
        line = bench_decode(args, dev, args.config)
    explicit = any(a == '--config' or a.startswith('--config=') for a in sys.argv[1:])
    if args.config == 'c2' and not explicit and not args.no_other_configs:
        # The other BASELINE configurations, measured in the same run (no CPU
        # baseline, 20 steps each), so that one default run records them all.
        sub = argparse.Namespace(**{**vars(args), 'steps': 20, 'warmup': 3, 'no_cpu_baseline': True,
                                    'ragged': False, 'head_dim': 128})
        line['other_configs'] = {name: _summary(fn()) for name, fn in (
            ('c3', lambda: bench_decode(sub, dev, 'c3')),
            ('c4', lambda: bench_mixed(sub, dev)),
            ('c5', lambda: bench_decode(sub, dev, 'c5')))}
    print(json.dumps(line), flush=True)


def _summary(line):
    keep = ('split_kernel_ms', 'merge_kernel_ms', 'prefill_kernel_ms', 'decode_ms', 'step_hbm_gbps')
    return {'workload': line['config']['workload'], 'value': line['value'], 'unit': line['unit'],
            'ms_per_step': line['ms_per_step'], 'dtype': line['dtype'],
            'roofline': {k: line['roofline'][k] for k in ('bound', 'achieved', 'peak', 'unit', 'frac', 'traffic')},
            **{k: line['config'][k] for k in keep if line['config'].get(k) is not None}}


def bench_decode(args, dev, config):
    """One decode configuration (C2, C3, C5 and their variants): the line for it."""
    from damendaemon_amd import kernels
    case, workload, dtype, nbytes = build_case(config, dev)
    launch = kernels.prepare_attention(case['query'], case['cache_k'], case['cache_v'], case['positions'],
                                       case['slots'], page_table=case['page_table'],
                                       k_scale=case.get('k_scale'), v_scale=case.get('v_scale'))
    for _ in range(args.warmup):
        launch.run()
    torch.cuda.synchronize()

    # Kernel timing: the split kernel and the merge bracketed by HIP events on
    # the launch stream (torch's current stream), K launches.
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for e0, e1, e2 in events:
        e0.record()
        launch.partials()
        e1.record()
        launch.merge()
        e2.record()
    torch.cuda.synchronize()
    split_ms = statistics.mean(e0.elapsed_time(e1) for e0, e1, _ in events)
    merge_ms = statistics.mean(e1.elapsed_time(e2) for _, e1, e2 in events)

    # Throughput: K steps (split kernel + merge) launched back to back on the
    # stream, as they run inside a model's forward pass, W untimed ones
    # first, exactly K timed between synchronisations (the host enqueues a
    # step in ~11 us, well ahead of the GPU).  The same step replayed alone
    # from a captured HIP graph (batch.py:25-46 captures the whole decode
    # forward) is reported beside it: each replay of a graph this small adds
    # a fixed gap of a few us before its first kernel.
    for _ in range(args.warmup):
        launch.run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        launch.run()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / args.steps * 1e3
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch.run()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    graph_ms = (time.perf_counter() - t0) / args.steps * 1e3
    batch = case['query'].shape[0]
    achieved = nbytes / (split_ms * 1e-3) / 1e9

    line = {
        'metric': 'paged decode attn tokens/s + achieved HBM GB/s (% peak), 1 MI355X',
        'value': batch / (ms_per_step * 1e-3),
        'unit': 'tokens/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': ms_per_step,
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': dtype,
        'data': 'synthetic (seeded N(0,1) Q/K/V, seeded page scatter)',
        'config': {'workload': workload, 'sequences': batch, 'context_tokens': sum(case['contexts']),
                   'splits': launch.splits, 'split_tokens': launch.split_tokens,
                   'split_kernel_ms': split_ms, 'merge_kernel_ms': merge_ms,
                   'step_hbm_gbps': nbytes / (ms_per_step * 1e-3) / 1e9,
                   'graph_replay_ms_per_step': graph_ms},
        'roofline': {'bound': 'hbm', 'achieved': achieved, 'peak': PEAK_HBM_GBPS, 'unit': 'GB/s',
                     'frac': achieved / PEAK_HBM_GBPS, 'traffic': measured_traffic(f'decode_{config}_pmc'),
                     'algorithmic_bytes': nbytes, 'source_digest': source_digest('decode')},
        'cpu_baseline': None if args.no_cpu_baseline else cpu_baseline(case),
    }
    return line


def bench_mixed(args, dev, dtype=torch.bfloat16):
    """Config C4: one step = GPU pack + K/V page write + mixed prefill/decode attention
    (c4f32: the same batch with fp32 pages, a float32 compute dtype)."""
    from damendaemon_amd import kernels, packing, ragged, workloads
    f32 = dtype == torch.float32
    peak = PEAK_FP32_TFLOPS if f32 else PEAK_BF16_TFLOPS
    D = args.head_dim
    case = workloads.config_c4(device=dev, dtype=dtype, dim=D)
    table, ck, cv = case['page_table'], case['cache_k'], case['cache_v']
    lengths, starts, slots = case['lengths'], case['starts'], case['seg_slots']
    n_chunks = sum(1 for n in lengths if n > 1)
    t_prefill = sum(lengths[:n_chunks])
    flops = 4 * 32 * D * sum(n * s + n * (n + 1) // 2 for n, s in zip(lengths[:n_chunks], starts[:n_chunks]))
    # decode rows where a streamed decode kernel exists (head sizes 64, 96,
    # 128, 256); at other head sizes the line times the prefill only
    decode_rows = D in (64, 96, 128, 256)

    def step(ev=None):
        packed = packing.pack_batch(lengths, starts, slots, table)
        packing.store_kv_pages(case['k_new'], case['v_new'], packed.slot_map, ck, cv)
        out = torch.empty_like(case['q'])
        # the host work of the prefill call (plan, upload) before the events,
        # so that they bracket the kernels only
        launch = ragged.prepare_prefill(case['q'], ck, cv, packed, table, out=out, segments=(0, n_chunks))
        if ev:
            ev[0].record()
        launch.phase(1)       # the attention kernel (the roofline's dominant kernel)
        if ev:
            ev[1].record()
        launch.phase(2)       # the bf16 exactness re-run: a near-empty launch on N(0,1) data
        if ev:
            ev[3].record()
        if decode_rows:
            kernels.prepare_attention(case['q'][t_prefill:].unsqueeze(2), ck, cv, packed.positions[t_prefill:],
                                      packed.slot_ids[t_prefill:], page_table=table,
                                      out=out[t_prefill:].unsqueeze(2)).run()
        if ev:
            ev[2].record()
        return out

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    t0 = time.perf_counter()
    for ev in events:
        step(ev)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    prefill_ms = statistics.mean(e[0].elapsed_time(e[1]) for e in events)
    rerun_ms = statistics.mean(e[1].elapsed_time(e[3]) for e in events)
    decode_ms = statistics.mean(e[3].elapsed_time(e[2]) for e in events) if decode_rows else None
    # --ragged: the same attention through ragged_attention, decode rows on a side stream beside the
    # prefill (kept out of the default run so that kernel traces show the kernels on their own)
    ragged_ms = None
    if args.ragged:
        packed = packing.pack_batch(lengths, starts, slots, table)
        ragged_ms = _event_mean_ms(lambda: ragged.ragged_attention(case['q'], ck, cv, packed, table), args.steps,
                                   args.warmup)
    tflops = flops / (prefill_ms * 1e-3) / 1e12
    ctx = [s + n for s, n in zip(starts, lengths)]
    decode_bytes = sum(ctx[n_chunks:]) * 8 * D * 2 * (4 if f32 else 2)
    ms = wall / args.steps * 1e3
    return {
        'metric': 'mixed chunked-prefill + decode attention: packed tokens/s, prefill MFMA utilisation, 1 MI355X',
        'value': sum(lengths) / (ms * 1e-3), 'unit': 'tokens/s', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': ms, 'higher_is_better': True, 'scaling': 'weak',
        'vs_baseline': None, 'dtype': 'f32' if f32 else 'bf16',
        'data': 'synthetic (seeded N(0,1) Q/K/V, seeded page scatter)',
        'config': {'workload': 'C4 mixed batch' + (' with fp32 pages' if f32 else '') +
                               ': 8 x 512-token chunks on contexts U[0,4096] + 120 decodes '
                               f'ctx U[256,8192], H32/KH8/D{D}, page 16 (GPU pack + page write + attention)',
                   'prefill_kernel_ms': prefill_ms, 'prefill_rerun_ms': rerun_ms, 'decode_ms': decode_ms,
                   'prefill_flops': flops,
                   'ragged_attention_ms': ragged_ms,
                   'decode_hbm_gbps': decode_bytes / (decode_ms * 1e-3) / 1e9 if decode_rows else None},
        'roofline': {'bound': 'mfma', 'achieved': tflops, 'peak': peak, 'unit': 'TFLOP/s',
                     'frac': tflops / peak,
                     'traffic': measured_traffic('prefill_c4_pmc', 'prefill') if not f32 and D == 128 else None},
        'cpu_baseline': None if args.no_cpu_baseline or not decode_rows else cpu_baseline_mixed(case, n_chunks)}


def _event_mean_ms(fn, steps, warmup):
    """Mean duration of fn's GPU work, HIP events on the launch stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    for a, b in events:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return statistics.mean(a.elapsed_time(b) for a, b in events)


def _hbm_line(metric, unit_value, unit, ms, nbytes, steps, warmup, dtype, workload, family, extra=None):
    achieved = nbytes / (ms * 1e-3) / 1e9
    return {'metric': metric, 'value': unit_value / (ms * 1e-3), 'unit': unit, 'n_gpus': 1, 'steps': steps,
            'warmup': warmup, 'ms_per_step': ms, 'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None,
            'dtype': dtype, 'data': 'synthetic (seeded)', 'config': dict({'workload': workload}, **(extra or {})),
            'roofline': {'bound': 'hbm', 'achieved': achieved, 'peak': PEAK_HBM_GBPS, 'unit': 'GB/s',
                         'frac': achieved / PEAK_HBM_GBPS, 'traffic': None, 'algorithmic_bytes': nbytes,
                         'source_digest': source_digest(family)},
            'cpu_baseline': None}


# The secondary HBM lines rotate over independent copies of their buffers so
# that no launch finds its inputs in the 256 MB Infinity Cache (MALL) left by
# the previous one: the sets together exceed it by far.
ROTATE = 4


def bench_rope(args, dev):
    """Fused RoPE + paged K/V write (kernels.rope_batch, reference kernels.py:271-340) on the
    C4 packed batch: 4,216 tokens, H32/KH8/D128 bf16, page 16.  Four independent copies of the
    batch (qkv rows, cos/sin tables, KV pools, page tables: ~3 GB each) are used in turn."""
    from damendaemon_amd import kernels, packing, workloads
    H, KH, D = 32, 8, 128
    sets = []
    for r in range(ROTATE):
        case = workloads.config_c4(device=dev, seed=4 + 11 * r)
        table, ck, cv = case['page_table'], case['cache_k'], case['cache_v']
        packed = packing.pack_batch(case['lengths'], case['starts'], case['seg_slots'], table)
        T = packed.total_tokens
        g = torch.Generator(device=dev).manual_seed(7 + r)
        qkv = torch.randn((T, (H + 2 * KH) * D), generator=g, device=dev).to(torch.bfloat16)
        positions_max = max(s + n for s, n in zip(case['starts'], case['lengths']))
        ang = torch.arange(positions_max, device=dev, dtype=torch.float32)[:, None] * \
            torch.pow(10000.0, -torch.arange(0, D, 2, device=dev, dtype=torch.float32) / D)[None, :]
        cos = torch.cat([ang.cos(), ang.cos()], 1).to(torch.bfloat16)
        sin = torch.cat([ang.sin(), ang.sin()], 1).to(torch.bfloat16)
        sets.append((qkv, cos, sin, packed, ck, cv, table))
        del case
    turn = [0]

    def step():
        qkv, cos, sin, packed, ck, cv, table = sets[turn[0] % ROTATE]
        turn[0] += 1
        kernels.rope_batch(qkv, cos, sin, packed.positions, packed.slot_ids, ck, cv, H, page_table=table)

    ms = _event_mean_ms(step, args.steps, args.warmup)
    T = sets[0][3].total_tokens
    # per token: qkv row read, cos + sin rows read, Q row written, K and V rows written into the
    # pages, position + slot ids, one page-table entry
    per_token = (H + 2 * KH) * D * 2 + 2 * D * 2 + H * D * 2 + 2 * KH * D * 2 + 16 + 4
    line = _hbm_line('fused RoPE + paged K/V write: tokens/s and achieved HBM GB/s (% peak), 1 MI355X', T,
                     'tokens/s', ms, T * per_token, args.steps, args.warmup, 'bf16',
                     'C4 packed batch through rope_batch: 4,216 tokens (8 x 512 prefill + 120 decode), '
                     'H32/KH8/D128, rotary dim 128, page 16; 4 independent batches used in turn', 'rope',
                     {'bytes_per_token': per_token, 'rotated_sets': ROTATE})
    line['roofline']['traffic'] = measured_traffic('rope_c4_kernel_trace', 'rope')
    return line


def bench_copy(args, dev):
    """copy_pages gather and restore (paged_kernels.copy_pages, reference paged_kernels.py:8-47) of one
    32,768-token slot of the C5 geometry: KH2/D256 bf16, pages scattered over the pool.  Four
    independent pools (84 MB each) and dense buffers (64 MB each) are used in turn."""
    from damendaemon_amd import paged_kernels
    KH, D, P, tokens = 2, 256, 16, 32768
    pages = tokens // P
    cap = pages + pages // 4
    sets = []
    for r in range(ROTATE):
        g = torch.Generator(device=dev).manual_seed(9 + r)
        cache = torch.randn((2, cap, KH, P, D), generator=g, device=dev).to(torch.bfloat16)
        perm = torch.randperm(cap, generator=torch.Generator().manual_seed(9 + r))[:pages]
        table = perm.to(torch.int32).reshape(1, pages).to(dev)
        dense = paged_kernels.copy_pages(cache, table, 0, tokens)
        sets.append((cache, table, dense))
    turn = [0]

    def gather():
        cache, table, _ = sets[turn[0] % ROTATE]
        turn[0] += 1
        paged_kernels.copy_pages(cache, table, 0, tokens)

    def restore():
        cache, table, dense = sets[turn[0] % ROTATE]
        turn[0] += 1
        paged_kernels.copy_pages(cache, table, 0, tokens, dense)

    gather_ms = _event_mean_ms(gather, args.steps, args.warmup)
    restore_ms = _event_mean_ms(restore, args.steps, args.warmup)
    dense = sets[0][2]
    nbytes = 2 * dense.numel() * dense.element_size() + pages * 4   # read + write, plus page-table entries
    line = _hbm_line('copy_pages gather: tokens/s and achieved HBM GB/s (% peak), 1 MI355X', tokens, 'tokens/s',
                     gather_ms, nbytes, args.steps, args.warmup, 'bf16',
                     'one 32,768-token slot, KH2/D256 bf16, page 16, pages scattered (C5 geometry); '
                     '4 independent pools used in turn', 'copy',
                     {'restore_ms': restore_ms, 'rotated_sets': ROTATE,
                      'restore_hbm_gbps': nbytes / (restore_ms * 1e-3) / 1e9})
    line['roofline']['traffic'] = measured_traffic('copy_pages_kernel_trace', 'copy')
    return line


if __name__ == '__main__':
    main()
