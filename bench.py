'''Benchmark of Motif Chord's sequence-mixing hot path on one MI355X.

Headline (value): config 3 -- full MotifChordModel forward at the 172M shape
(d=768, 4 blocks x (3 GDN + 1 Chord), H=12, GDN dk=64 / dv=128, Chord D=64 /
Hkv=3, SwiGLU 2048, vocab 32000), B=1, T=4096, bf16, random init
(Linear / Embedding / Conv1d ~ N(0, 0.02), semantic parameters at their
constructor values), uniform random token ids.  One step = one forward pass
(logits included), captured once as a hipGraph and replayed (every kernel runs
each step; the replayed logits are checked equal to an eager forward's); value =
tokens / s.  The eager (Python-launched) forward is reported beside it.

Also reported in the same JSON line:
- decode (config 4): one decode step at B=64 over a 4096-token context
  (KV caches and recurrent states filled with random values; labelled), as a
  captured hipGraph replayed K times;
- per-kernel timings of the hot-path ops at the config-3/4 shapes with HIP
  events on the launch stream (forward and backward), and the roofline of the
  dominant kernel;
- cpu_baseline: this build's CPU restatement of the reference's PyTorch path
  (oracle/, float32, torch threads) on config-3 forwards (1 warm-up, median of
  3); the config rows carry the same for configs 1, 2, 4 and a config-5 subset.

Usage: python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--no-cpu]
       python bench.py --kernels-only   # hot-path ops + a copy of known size and the peak
                                        # probes: the target of the rocprofv3 --pmc runs
'''
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, 'codon-motif_amd')):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = 'prefill tok/s @T=4096 + decode tok/s @B=64; % MFMA / HBM roofline (1 GPU)'
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def bench_config(vocab=32000):
    from motif.model.presets import config_172m
    return config_172m(vocab)


def init_model(model, std=0.02, seed=0):
    from motif.model.presets import init_random
    return init_random(model, std, seed)


def cuda_time(fn, steps, warmup):
    '''Average milliseconds of fn() over `steps` launches, HIP events on the current stream.'''
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def op_time(fn, launches, replays=5):
    '''Average device milliseconds of one fn() launch: `launches` calls captured in one
    hipGraph, replayed `replays` times between HIP events on the capturing stream, so
    host launch overhead does not enter the figure (it matches the rocprofv3 kernel
    durations of the same op).'''
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(launches):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (replays * launches)


def kernel_timings(dev):
    '''Hot-path ops at the config-3 / config-4 shapes.'''
    import torch
    import torch.nn.functional as F

    import motif.ops as ops
    from motif.ops.gated_deltanet import gdn_recurrent_into
    from oracle.chord import chord_prefill_flops
    from oracle.gdn import gdn_prefill_flops

    g = torch.Generator().manual_seed(0)
    res = {}
    B, H, T, dk, dv = 1, 12, 4096, 64, 128
    q = F.normalize(torch.randn(B, T, H, dk, generator=g), dim=-1).transpose(1, 2).to(dev, torch.bfloat16)
    k = F.normalize(torch.randn(B, T, H, dk, generator=g), dim=-1).transpose(1, 2).to(dev, torch.bfloat16)
    v = torch.randn(B, T, H, dv, generator=g).transpose(1, 2).to(dev, torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g)).transpose(1, 2).to(dev, torch.bfloat16)
    gg = F.logsigmoid(torch.randn(B, T, H, generator=g)).transpose(1, 2).to(dev, torch.bfloat16)
    ms = op_time(lambda: ops.chunk_gated_delta_rule(q, k, v, beta, gg), 20)
    fl = gdn_prefill_flops(B, T, H, dk, dv)
    res['gdn_chunk_prefill'] = dict(us=ms * 1e3, unit='TFLOP/s', achieved=fl / (ms * 1e-3) / 1e12,
                                    peak=PEAK_BF16_TFLOPS, bound='mfma', work=fl,
                                    shape='B=1 H=12 T=4096 dk=64 dv=128 bf16')

    Hc, Hkv, D = 12, 3, 64
    qc = (torch.randn(1, T, Hc, D, generator=g) * 0.5).transpose(1, 2).to(dev, torch.bfloat16)
    kc = (torch.randn(1, T, Hkv, D, generator=g) * 0.5).transpose(1, 2).to(dev, torch.bfloat16)
    vc = (torch.randn(1, T, Hkv, D, generator=g) * 0.5).transpose(1, 2).to(dev, torch.bfloat16)
    al = (torch.randn(Hc, generator=g) * 0.1).to(dev)
    be = (torch.randn(Hc, generator=g) * 0.1).to(dev)
    mu = torch.zeros(Hc, device=dev)
    ss = torch.ones(Hc, device=dev)
    ln = torch.log(torch.arange(1, T + 1, dtype=torch.float32, device=dev))[None].contiguous()
    ms = op_time(lambda: ops.apply_chord_attention(qc, kc, vc, al, be, mu, ss, ln, q_start=0), 20)
    fl = chord_prefill_flops(1, Hc, D, T)
    res['chord_prefill'] = dict(us=ms * 1e3, unit='TFLOP/s', achieved=fl / (ms * 1e-3) / 1e12,
                                peak=PEAK_BF16_TFLOPS, bound='mfma', work=fl,
                                shape='B=1 H=12 Hkv=3 T=4096 D=64 bf16 causal')

    # fused single-token GDN layer step (conv + norms + gates + delta rule + GatedRMSNorm),
    # from the fused projection row to the o_proj input, state and conv tails in place
    Bd, K = 64, 4
    hk, hv = H * dk, H * dv
    ncols = 2 * hk + 2 * hv + 2 * H
    offs = (0, hk, 2 * hk, 2 * hk + hv, 2 * hk + 2 * hv, 2 * hk + 2 * hv + H)
    proj = (torch.randn(Bd, ncols, generator=g) * 0.5).to(dev, torch.bfloat16)
    cw = [(torch.randn(c, 1, K, generator=g) * 0.3).to(dev, torch.bfloat16) for c in (hk, hk, hv)]
    tails = [(torch.randn(Bd, c, K - 1, generator=g) * 0.5).to(dev, torch.bfloat16) for c in (hk, hk, hv)]
    a_log = torch.empty(H).uniform_(1, 16, generator=g).log().to(dev, torch.bfloat16)
    dt_bias = (torch.rand(H, generator=g) * 0.1).to(dev, torch.bfloat16)
    nw = torch.ones(dv, device=dev, dtype=torch.bfloat16)
    # cache-cold: the launches rotate over 12 state / tail sets (302 MB, more than the
    # 256 MB last-level cache), as the 12 GDN layers of a decode step do
    n_sets = 12
    S0 = (torch.randn(Bd, H, dk, dv, generator=g) * 0.05).to(dev)
    Ss = [S0.clone() for _ in range(n_sets)]
    tls = [[t.clone() for t in tails] for _ in range(n_sets)]
    turn = [0]

    def gdn_step():
        i = turn[0] % n_sets
        turn[0] += 1
        ops.gdn_decode_fused(proj, offs, cw, tls[i], a_log, dt_bias, nw, 1e-6, Ss[i], H, dk, dv)
    ms = op_time(gdn_step, 48)
    byts = (Bd * H * dk * dv * 4 * 2                      # state read + write
            + Bd * (2 * hk + hv) * (K - 1) * 2 * 2        # conv tails read + write
            + Bd * ncols * 2 + (2 * hk + hv) * K * 2      # projections, conv weights
            + Bd * hv * 2)                                # output
    res['gdn_decode'] = dict(us=ms * 1e3, unit='GB/s', achieved=byts / (ms * 1e-3) / 1e9,
                             peak=PEAK_HBM_GBS, bound='hbm', work=byts,
                             shape='B=64 H=12 dk=64 dv=128 K=4, fused layer step, fp32 state in place; '
                                   'cache-cold (12 rotating state sets)')
    del Ss, tls

    Sk = 4097
    qk = (torch.randn(Bd, Hc, 1, D, generator=g) * 0.5).to(dev, torch.bfloat16)
    kk = (torch.randn(Bd, Hkv, Sk, D, generator=g) * 0.5).to(dev, torch.bfloat16)
    vk = (torch.randn(Bd, Hkv, Sk, D, generator=g) * 0.5).to(dev, torch.bfloat16)
    lnd = torch.full((Bd, 1), float(torch.log(torch.tensor(float(Sk)))), device=dev)
    # cache-cold: four K / V sets (805 MB) in rotation, as the 4 Chord layers of a step
    kvs = [(kk, vk)] + [(kk.clone(), vk.clone()) for _ in range(3)]
    turn = [0]

    def chord_step():
        kx, vx = kvs[turn[0] % len(kvs)]
        turn[0] += 1
        ops.apply_chord_attention(qk, kx, vx, al, be, mu, ss, lnd)
    ms = op_time(chord_step, 20)
    byts = 2 * Bd * Hkv * Sk * D * 2 + 2 * Bd * Hc * D * 2
    res['chord_decode'] = dict(us=ms * 1e3, unit='GB/s', achieved=byts / (ms * 1e-3) / 1e9,
                               peak=PEAK_HBM_GBS, bound='hbm', work=byts,
                               shape='B=64 H=12 Hkv=3 S=4097 D=64 bf16 (split-K + merge); cache-cold '
                                     '(4 rotating K / V sets)')
    del kvs

    # backward passes at the config-3 layer shape (eager launches, HIP events): the GDN chunk
    # rule in fp32 (per-chunk kernels + the two scans) and the Chord op in bf16
    from motif.ops.gdn_grad import _backward_kernels
    qf, kf, vf, bf_, gf = (t.float() for t in (q, k, v, beta, gg))
    dof = torch.randn(B, H, T, dv, generator=g).to(dev)
    dSf = (torch.randn(B, H, dk, dv, generator=g) * 0.1).to(dev)
    ms = cuda_time(lambda: _backward_kernels(qf, kf, vf, bf_, gf, None, dof, dSf, 64), 10, 3)
    res['gdn_chunk_backward'] = dict(us=ms * 1e3, shape='B=1 H=12 T=4096 dk=64 dv=128 fp32 (the chunk rule\'s '
                                                      'gradients: per-chunk kernels and the two scans)')
    with torch.enable_grad():
        qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (qc, kc, vc))
        out = ops.apply_chord_attention(qg, kg, vg, al, be, mu, ss, ln, q_start=0)
        dob = torch.randn(out.shape, generator=g).to(dev, torch.bfloat16)
        ms = cuda_time(lambda: torch.autograd.grad(out, (qg, kg, vg), dob, retain_graph=True), 10, 3)
    res['chord_backward'] = dict(us=ms * 1e3, forward_us=res['chord_prefill']['us'],
                                 shape='B=1 H=12 Hkv=3 T=4096 D=64 bf16 causal (dQ, dK, dV)')
    for r in res.values():
        if 'peak' in r:
            r['frac'] = r['achieved'] / r['peak']
    return res


def _median_ms(fn, reps=10):
    '''Median device milliseconds of fn() over `reps` launches, one HIP event pair each.'''
    import torch
    fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    return sorted(ts)[len(ts) // 2]


def measured_peaks(dev):
    '''The roofline denominators measured on this GPU (median of 10 launches each):
    a 1 GiB device copy (2 GiB of traffic), a 2 GiB read-only reduction and a loop of
    independent dense bf16 MFMAs (motif_probe_* in codon-motif_amd/csrc/peaks.hip).'''
    import torch

    from motif.ops import _lib
    lib = _lib.lib()
    st = _lib.stream_ptr(dev)
    ncu = torch.cuda.get_device_properties(dev).multi_processor_count
    src = torch.ones(2 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    red = torch.empty(32 * ncu, dtype=torch.int32, device=dev)

    def run(rc, what):
        _lib.check(rc, what)

    copy_ms = _median_ms(lambda: run(lib.motif_probe_copy(src.data_ptr(), dst.data_ptr(), 1 << 30, 16 * ncu, st),
                                     'motif_probe_copy'))
    read_ms = _median_ms(lambda: run(lib.motif_probe_read(src.data_ptr(), red.data_ptr(), 2 << 30, 32 * ncu, st),
                                     'motif_probe_read'))
    grid, iters = 8 * ncu, 2048
    out = torch.empty(grid * 256, dtype=torch.float32, device=dev)
    rates = {}
    for shape, per in ((16, 8 * 16384), (32, 4 * 32768)):
        ms = _median_ms(lambda: run(lib.motif_probe_mfma_bf16(out.data_ptr(), grid, iters, shape, st),
                                    'motif_probe_mfma_bf16'))
        rates[shape] = grid * 4 * iters * per / (ms * 1e-3) / 1e12
    del src, dst, red, out
    return {'hbm_copy_GBs': round(2 * 2 ** 30 / (copy_ms * 1e-3) / 1e9, 1),
            'hbm_read_GBs': round(2 * 2 ** 30 / (read_ms * 1e-3) / 1e9, 1),
            'mfma_bf16_TFLOPs': round(max(rates.values()), 1),
            'mfma_bf16_16x16x32_TFLOPs': round(rates[16], 1), 'mfma_bf16_32x32x16_TFLOPs': round(rates[32], 1),
            'published': {'hbm_GBs': PEAK_HBM_GBS, 'mfma_bf16_TFLOPs': PEAK_BF16_TFLOPS},
            'method': '1 GiB copy (bytes read + written; a contiguous block per workgroup), 2 GiB read-only '
                      'reduction, both with nontemporal 16-byte accesses, 8 in flight per thread; '
                      f'{grid} workgroups x 4 waves x {iters} rounds of 8 independent '
                      'v_mfma_f32_16x16x32_bf16 or 4 independent v_mfma_f32_32x32x16_bf16; '
                      'median of 10 launches each'}


def _cpu_time(fn, reps=3):
    '''Seconds per call of fn on the host threads: one untimed warm-up call, then the median
    of `reps` timed calls.'''
    import torch
    torch.set_num_threads(os.cpu_count() or 1)
    times = []
    with torch.no_grad():
        fn()
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def config_rows(dev, model, with_cpu=True):
    '''The other configurations of the scope table at their own shapes: config 1 (GDN op,
    fp32), config 2 (Chord op, bf16, Hkv 12 and 3) and, for the CPU baseline only,
    config 4 (decode steps of the oracle model on random-filled caches).  GPU figures are
    op_time averages (graph-replayed launches); CPU figures the oracle's median of 3 runs
    after a warm-up (config 5: the two shortest sequences, extrapolated per token).'''
    import torch
    import torch.nn.functional as F

    import motif.ops as ops
    from oracle.chord import chord_attention, chord_prefill_flops
    from oracle.gdn import chunked, gdn_prefill_flops
    rows = {}

    # config 1: B=1 H=4 T=256 dk=dv=64 fp32, q / k L2-normalised
    g = torch.Generator().manual_seed(0)
    B, H, T, dk, dv = 1, 4, 256, 64, 64
    q = F.normalize(torch.randn(B, H, T, dk, generator=g), dim=-1)
    k = F.normalize(torch.randn(B, H, T, dk, generator=g), dim=-1)
    v = torch.randn(B, H, T, dv, generator=g)
    beta = torch.sigmoid(torch.randn(B, H, T, generator=g))
    gg = F.logsigmoid(torch.randn(B, H, T, generator=g))
    dq, dk_, dv_, db, dg = (t.to(dev) for t in (q, k, v, beta, gg))
    ms = op_time(lambda: ops.chunk_gated_delta_rule(dq, dk_, dv_, db, dg), 20)
    fl = gdn_prefill_flops(B, T, H, dk, dv)
    rows['config1_gdn_chunk_fp32'] = {
        'shape': 'B=1 H=4 T=256 dk=dv=64 fp32', 'gpu_us': round(ms * 1e3, 2),
        'gpu_tok_s': round(B * T / (ms * 1e-3), 1), 'flops': fl}
    if with_cpu:
        dt = _cpu_time(lambda: chunked(q, k, v, beta, gg))
        rows['config1_gdn_chunk_fp32']['cpu_oracle_us'] = round(dt * 1e6, 1)

    # config 2: B=2 H=12 T=2048 D=64 bf16, Hkv 12 (the configuration) and 3 (the model's)
    Bc, Hc, Tc, D = 2, 12, 2048, 64
    al = torch.randn(Hc, generator=g) * 0.1
    be = torch.randn(Hc, generator=g) * 0.1
    mu, ss = torch.zeros(Hc), torch.ones(Hc)
    ln = torch.log(torch.arange(1, Tc + 1, dtype=torch.float32))[None].expand(Bc, Tc).contiguous()
    fl = chord_prefill_flops(Bc, Hc, D, Tc)
    for hkv in (12, 3):
        qc = (torch.randn(Bc, Hc, Tc, D, generator=g) * 0.5).to(torch.bfloat16)
        kc = (torch.randn(Bc, hkv, Tc, D, generator=g) * 0.5).to(torch.bfloat16)
        vc = (torch.randn(Bc, hkv, Tc, D, generator=g) * 0.5).to(torch.bfloat16)
        args = [t.to(dev) for t in (qc, kc, vc, al, be, mu, ss, ln)]
        ms = op_time(lambda: ops.apply_chord_attention(*args, q_start=0), 20)
        r = {'shape': f'B=2 H=12 Hkv={hkv} T=2048 D=64 bf16 causal', 'gpu_us': round(ms * 1e3, 2),
             'gpu_TFLOPs': round(fl / (ms * 1e-3) / 1e12, 2), 'frac_of_published_mfma':
             round(fl / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4), 'flops': fl}
        if with_cpu and hkv == 12:
            dt = _cpu_time(lambda: chord_attention(qc.float(), kc.float(), vc.float(), al, be, mu, ss, ln,
                                                   q_start=0, compute_dtype=torch.float32))
            r['cpu_oracle_us'] = round(dt * 1e6, 1)
        rows[f'config2_chord_prefill_hkv{hkv}'] = r

    # config 4 on the CPU: decode steps of the oracle model over random-filled caches
    if with_cpu:
        from oracle.model import OracleModel
        cfg = model.config
        p = {kk: vv.detach().float().cpu() for kk, vv in model.state_dict().items()}
        om = OracleModel(p, dict(model_dim=cfg.model_dim, num_heads=cfg.num_heads, num_kv_heads=cfg.num_kv_heads,
                                 head_k_dim=cfg.head_k_dim, block=cfg.block, block_n=cfg.block_n),
                         dtype=torch.float32)
        Bd, ctx, hd = 64, 4096, cfg.model_dim // cfg.num_heads
        gd = torch.Generator().manual_seed(1)
        for li, kind in enumerate(list(cfg.block) * cfg.block_n):
            if kind == 'chord':
                om.kc[li] = torch.randn(Bd, cfg.num_kv_heads, ctx, hd, generator=gd) * 0.5
                om.vc[li] = torch.randn(Bd, cfg.num_kv_heads, ctx, hd, generator=gd) * 0.5
            else:
                om.state[li] = torch.randn(Bd, om.H, om.dk, om.dv, generator=gd) * 0.05
                om.conv[li] = tuple(torch.randn(Bd, c, 3, generator=gd) * 0.5
                                    for c in (om.H * om.dk, om.H * om.dk, om.H * om.dv))
        om.pos = ctx
        ids = torch.randint(0, cfg.vocab_size, (Bd, 1), generator=gd)
        dt = _cpu_time(lambda: om.forward(ids))
        rows['config4_decode_cpu'] = {
            'shape': 'B=64, context 4096 (random-filled caches), one token per step', 'cpu_oracle_ms_per_step':
            round(dt * 1e3, 1), 'cpu_tok_s': round(Bd / dt, 1), 'cores': torch.get_num_threads(),
            'method': '1 warm-up step, median of 3 steps (the context grows by one per step)'}
    rows['config5_packed_prefill'] = {
        'skipped': 'the packed route is kept off the GPU at this size: a packed 73364-token prefill exceeded its '
                   'test time limit with the fused GatedDelta front end (now switched off for packed input); '
                   'cause not established',
        'gpu_per_sequence': config5_per_sequence(dev, model)}
    if with_cpu:
        rows['config5_packed_prefill']['cpu'] = config5_cpu_subset(model)
    return rows


def config5_per_sequence(dev, model, reps=3):
    '''Config 5's workload on the GPU through the unpacked route: each of the 16
    sequences (lengths from presets.packed_lengths(), ids seeded as the packed test's) is
    one B = 1 forward from empty state, logits included, captured as its own hipGraph;
    a round replays the 16 graphs in order between HIP events; 1 warm-up round, median
    of `reps`.  tok/s = 73364 tokens / round time.'''
    import torch

    from motif.model.presets import cu_seqlens_of, packed_lengths
    lens = packed_lengths()
    cu = cu_seqlens_of(lens).tolist()
    ids = torch.randint(0, model.config.vocab_size, (1, cu[-1]), generator=torch.Generator().manual_seed(5))
    seqs = [ids[:, a:b].to(dev) for a, b in zip(cu[:-1], cu[1:])]
    graphs = []
    side = torch.cuda.Stream()
    for s in seqs:
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            model(s)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = model(s)
        graphs.append((g, out))
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for r in range(reps + 1):
        torch.cuda.synchronize()
        ev0.record()
        for g, _ in graphs:
            g.replay()
        ev1.record()
        torch.cuda.synchronize()
        if r:
            times.append(ev0.elapsed_time(ev1))
    finite = all(bool(torch.isfinite(out.logits).all()) for _, out in graphs)
    del graphs
    ms = sorted(times)[len(times) // 2]
    return {'route': 'each sequence as its own B=1 forward from empty state (unpacked kernels), one hipGraph per '
                     'sequence, the 16 replayed in order; 1 warm-up round, median of '
                     f'{reps}', 'tokens': cu[-1], 'ms': round(ms, 3), 'tok_s': round(cu[-1] / (ms * 1e-3), 1),
            'logits_finite': finite}


def config5_cpu_subset(model, n=2):
    '''Config 5 on the CPU: the n shortest of the 16 packed sequences through the oracle
    model one at a time (each from zero state, as packing makes them), 1 warm-up + median of
    3, and the whole 73364-token workload extrapolated per token from that sample.'''
    import torch

    from motif.model.presets import packed_lengths
    from oracle.model import OracleModel
    cfg = model.config
    p = {kk: vv.detach().float().cpu() for kk, vv in model.state_dict().items()}
    ocfg = dict(model_dim=cfg.model_dim, num_heads=cfg.num_heads, num_kv_heads=cfg.num_kv_heads,
                head_k_dim=cfg.head_k_dim, block=cfg.block, block_n=cfg.block_n)
    lens = packed_lengths()
    pick = sorted(range(len(lens)), key=lambda i: lens[i])[:n]
    g = torch.Generator().manual_seed(5)
    seqs = [torch.randint(0, cfg.vocab_size, (1, lens[i]), generator=g) for i in pick]
    om = OracleModel(p, ocfg, dtype=torch.float32)

    def run():
        for s in seqs:
            om.reset()
            om.forward(s)
    dt = _cpu_time(run)
    tokens = sum(lens[i] for i in pick)
    tok_s = tokens / dt
    return {'sample': f'sequences {pick} (lengths {[lens[i] for i in pick]}) of the 16, through oracle/ in float32 '
                      f'one at a time; 1 warm-up, median of 3', 'cpu_tok_s': round(tok_s, 1),
            'cores': torch.get_num_threads(), 'extrapolated_s_all_16': round(sum(lens) / tok_s, 1),
            'note': 'extrapolated per token from the shortest sequences: the attention cost per token grows '
                    'with length, so the full run would take longer'}


def copy_calibration(dev, mib=256, reps=5):
    '''A plain device copy of `mib` MiB (reads and writes exactly that many bytes):
    the scale for the FETCH_SIZE / WRITE_SIZE counters of the --pmc runs.'''
    import torch
    src = torch.ones(mib * 2 ** 19, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    return mib * 1024  # KiB per direction


# rocprofv3 --pmc summary (FETCH_SIZE / WRITE_SIZE, copy-calibrated) of bench.py --kernels-only
TRAFFIC_FILE = os.path.join(ROOT, 'profiles', 'hot_path_ops_hbm_traffic.txt')
OP_KERNELS = {'gdn_chunk_prefill': ('gdn_prep_mfma', 'gdn_state_scan', 'gdn_chunk_out'),
              'chord_prefill': ('chord_fwd_kernel',),
              'gdn_decode': ('gdn_decode_kernel',),
              'chord_decode': ('chord_decode_mfma_kernel', 'chord_merge_kernel')}


def measured_traffic(op):
    '''HBM bytes per launch of `op` (all its kernels) from the committed --pmc summary, or None.'''
    try:
        with open(TRAFFIC_FILE) as f:
            rows = [ln.split() for ln in f
                    if ln[:1].isalpha() and len(ln.split()) == 5 and ln.split()[1].isdigit()]
    except OSError:
        return None
    total, seen = 0.0, set()
    for r in rows:
        name = r[0].split('<')[0]
        if name in OP_KERNELS.get(op, ()):
            total += float(r[4]) * 1e6
            seen.add(name)
    return total if seen == set(OP_KERNELS.get(op, ())) else None


def make_decode_cache(model, B, ctx, capacity, dev, dtype, seed=1):
    '''Fixed-capacity caches as after a ctx-token prefill, filled with random values
    (timing only): keys / values ~ 0.5 N(0, 1), states ~ 0.05 N(0, 1), tails ~ 0.5 N(0, 1).'''
    import torch

    from motif.model.cache import ModelCache, StaticKVLayerCache
    g = torch.Generator().manual_seed(seed)
    cache = ModelCache.for_decode(model, B, capacity, dev, dtype)
    for lc in cache.layer_caches():
        if isinstance(lc, StaticKVLayerCache):
            shape = (B, lc._slab[0].shape[1], ctx, lc._slab[0].shape[3])
            lc.fill((torch.randn(shape, generator=g) * 0.5).to(dev, dtype),
                    (torch.randn(shape, generator=g) * 0.5).to(dev, dtype))
        else:
            lc.state.copy_(torch.randn(lc.state.shape, generator=g) * 0.05)
            for t in lc.conv_state:
                t.copy_(torch.randn(t.shape, generator=g) * 0.5)
            lc.length = ctx
    for b in cache.blocks:
        b.attn_res.seq_len = ctx
    return cache


def cpu_baseline(T=4096, seed=0):
    '''Config-3 forwards through the CPU oracle (float32) on the host threads: 1 warm-up,
    then the median of 3.'''
    import torch

    from motif.model.motif import MotifChordModel
    from oracle.model import OracleModel
    cfg = bench_config()
    model = init_model(MotifChordModel(cfg), seed=seed)
    p = {k: v.detach().float() for k, v in model.state_dict().items()}
    ocfg = dict(model_dim=cfg.model_dim, num_heads=cfg.num_heads, num_kv_heads=cfg.num_kv_heads,
                head_k_dim=cfg.head_k_dim, block=cfg.block, block_n=cfg.block_n)
    om = OracleModel(p, ocfg, dtype=torch.float32)
    ids = torch.randint(0, cfg.vocab_size, (1, T), generator=torch.Generator().manual_seed(seed))
    dt = _cpu_time(lambda: (om.reset(), om.forward(ids)))
    cpu_model = ''
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    cpu_model = line.split(':', 1)[1].strip()
                    break
    except OSError:
        pass
    return dict(value=T / dt, unit='tok/s', cores=torch.get_num_threads(), kind='port',
                sample=f'config-3 forward (B=1, T={T}) through oracle/ (CPU restatement of the '
                       f'reference torch path: chunk loop GDN, eager Chord), float32; 1 warm-up, median '
                       f'of 3: {dt:.2f} s per forward; CPU: {cpu_model}')


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=10)
    ap.add_argument('--warmup', type=int, default=3)
    ap.add_argument('--no-cpu', action='store_true')
    ap.add_argument('--kernels-only', action='store_true')
    ap.add_argument('--seq', type=int, default=4096)
    ap.add_argument('--decode-batch', type=int, default=64)
    args = ap.parse_args()
    world = int(os.environ.get('WORLD_SIZE', '1'))
    if args.gpus != 1 or world != 1:
        print(f'bench.py measures one GPU only (this build has no multi-GPU path); '
              f'got --gpus {args.gpus}, WORLD_SIZE={world}', file=sys.stderr)
        sys.exit(2)

    import torch

    import motif.ops as ops
    from motif.model.motif import MotifChordModel
    if not ops.HAS_TRITON:
        raise RuntimeError('HIP kernel library not loaded or no ROCm device visible')
    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    torch.backends.cuda.matmul.allow_tf32 = False
    from motif import tuning
    tuned = tuning.enable()
    log(f'[bench] library GEMM tuning results loaded: {tuned}')

    if args.kernels_only:
        with torch.no_grad():
            kern = kernel_timings(dev)
            copy_calibration(dev)
            # the probes of known rate: the copy scales the traffic counters, the MFMA
            # loop marks a fully busy matrix pipe for the MFMA-busy counter
            kern['peaks'] = measured_peaks(dev)
        print(json.dumps({k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                          for k, v in kern.items()}), flush=True)
        return

    cfg = bench_config()
    model = init_model(MotifChordModel(cfg)).to(dev, torch.bfloat16).eval()
    T = args.seq
    ids = torch.randint(0, cfg.vocab_size, (1, T), generator=torch.Generator().manual_seed(0)).to(dev)

    log(f'[bench] prefill B=1 T={T}: warmup {args.warmup}, steps {args.steps}')
    with torch.no_grad():
        for _ in range(args.warmup):
            model(ids)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(args.steps):
            model(ids)
        ev1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms_eager = ev0.elapsed_time(ev1) / args.steps
    log(f'[bench] prefill (eager) {ms_eager:.2f} ms/step ({T / (ms_eager * 1e-3):.0f} tok/s, wall {wall:.2f} s)')

    # The same forward captured once as a hipGraph and replayed: every kernel runs every
    # step (nothing cached between replays); host launch gaps between the ~290 kernels
    # are gone.  This is the headline figure; the eager one is reported beside it.
    log('[bench] prefill as a captured hipGraph')
    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            model(ids)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        pgraph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(pgraph):
            pout = model(ids)
        for _ in range(args.warmup):
            pgraph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record()
        for _ in range(args.steps):
            pgraph.replay()
        ev1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        # the replayed logits equal an eager forward's
        eager_logits = model(ids).logits
        graph_ok = bool(torch.equal(pout.logits, eager_logits))
    ms_step = ev0.elapsed_time(ev1) / args.steps
    prefill_tok_s = T / (ms_step * 1e-3)
    with torch.no_grad():
        pre_med = _median_ms(pgraph.replay, reps=max(args.steps, 10))
    log(f'[bench] prefill (graph) {ms_step:.2f} ms/step ({prefill_tok_s:.0f} tok/s, wall {wall:.2f} s), '
        f'logits equal eager: {graph_ok}')
    del pgraph, pout, eager_logits

    log('[bench] decode B=64 ctx=4096 (one captured step replayed token after token)')
    from motif.model.decode_graph import DecodeGraph
    Bd, ctx = args.decode_batch, 4096
    n_dec = max(args.steps * 10, 100)
    cache = make_decode_cache(model, Bd, ctx, ctx + 2 * n_dec + 16, dev, torch.bfloat16)
    toks = torch.randint(0, cfg.vocab_size, (n_dec + 8, Bd, 1), generator=torch.Generator().manual_seed(1)).to(dev)
    with torch.no_grad():
        graph = DecodeGraph(model, cache, Bd)
        for i in range(3):
            graph.step(toks[i])
        torch.cuda.synchronize()
        ev0.record()
        for i in range(n_dec):
            graph.step(toks[3 + i])
        ev1.record()
        torch.cuda.synchronize()
    dec_ms = ev0.elapsed_time(ev1) / n_dec
    decode_tok_s = Bd / (dec_ms * 1e-3)
    with torch.no_grad():
        dec_med = _median_ms(graph.step, reps=n_dec)
    log(f'[bench] decode {dec_ms:.3f} ms/step ({decode_tok_s:.0f} tok/s), context {ctx} -> {cache.seq_len}')
    del graph, cache

    log('[bench] kernel timings')
    with torch.no_grad():
        kern = kernel_timings(dev)
    for name, r in kern.items():
        if 'frac' in r:
            log(f'[bench]   {name}: {r["us"]:.1f} us, {r["achieved"]:.1f} {r["unit"]} ({100 * r["frac"]:.1f}% of peak)')
        else:
            log(f'[bench]   {name}: {r["us"]:.1f} us')
    # the dominant prefill kernel: the one that takes the most time per forward
    per_fwd = {'gdn_chunk_prefill': kern['gdn_chunk_prefill']['us'] * 12,
               'chord_prefill': kern['chord_prefill']['us'] * 4}
    dom = max(per_fwd, key=per_fwd.get)
    r = kern[dom]
    log('[bench] measured peaks')
    with torch.no_grad():
        peaks = measured_peaks(dev)
    log(f'[bench]   {peaks}')
    mpeak = peaks['mfma_bf16_TFLOPs'] if r['bound'] == 'mfma' else peaks['hbm_copy_GBs']
    roofline = dict(kernel=dom, bound=r['bound'], achieved=round(r['achieved'], 3), peak=r['peak'],
                    unit=r['unit'], frac=round(r['frac'], 5), traffic=measured_traffic(dom), avg_us=round(r['us'], 2),
                    work_per_launch=r['work'], shape=r['shape'], measured_peak=mpeak,
                    frac_of_measured=round(r['achieved'] / mpeak, 5))
    log('[bench] configs 1, 2 (GPU ops) and CPU baselines of configs 1, 2, 4')
    with torch.no_grad():
        configs = config_rows(dev, model, with_cpu=not args.no_cpu)
    for name, row in configs.items():
        log(f'[bench]   {name}: {row}')

    cpu = None
    if not args.no_cpu:
        log('[bench] cpu baseline (oracle, float32, one T=4096 forward)')
        cpu = cpu_baseline(T)
        log(f'[bench] cpu {cpu["value"]:.1f} tok/s on {cpu["cores"]} threads')

    line = {
        'metric': METRIC, 'value': round(prefill_tok_s, 1), 'unit': 'tok/s', 'n_gpus': 1,
        'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': round(ms_step, 4),
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16',
        'data': 'synthetic (uniform random ids; random-init weights of the 172M-shape architecture)',
        'config': {'workload': 'config 3: MotifChordModel forward, d=768, 4x(3 GDN + 1 Chord), H=12, '
                               'GDN dk=64 dv=128, Chord D=64 Hkv=3, vocab 32000, B=1, T=4096, bf16',
                   'global_batch': 1, 'seq_len': T, 'parallelism': 'single GPU',
                   'execution': 'forward captured once as a hipGraph, replayed per step (inside the graph '
                                'each decoder\'s MLP branch runs on a second stream beside its attention layer)'},
        'prefill_eager': {'tok_s': round(T / (ms_eager * 1e-3), 1), 'ms_per_step': round(ms_eager, 4),
                          'note': 'the same forward launched from Python each step'},
        'prefill_graph_matches_eager': graph_ok,
        'prefill_median_ms': round(pre_med, 4),
        'decode': {'tok_s': round(decode_tok_s, 1), 'ms_per_step': round(dec_ms, 4),
                   'median_ms_per_step': round(dec_med, 4), 'batch': Bd,
                   'context': ctx, 'steps': n_dec,
                   'note': 'config 4: one decode step captured as a hipGraph and replayed token after token '
                           '(device-resident cache cursors, no host rewinds; the context grows from 4096 by one '
                           'position per step); caches random-filled to 4096 positions (timing only)'},
        'roofline': roofline,
        'peaks': peaks,
        'configs': configs,
        'kernels': {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in kern.items()},
        'cpu_baseline': cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
