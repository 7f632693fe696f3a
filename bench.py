#!/usr/bin/env python3
"""Benchmark of the Bifrost core on one MI355X.

Headline workload (one step = one pass of the hot path over one batch of synthetic input): the converted (Bifrost)
layer's prefill at 32K, i.e. ``_student`` over a 32768-token chunk from an empty cache: B=1, T=32768, H=24 query
heads, G=4 KV heads, D=256, window 2048 + 4 sinks, bf16 activations, fp32 delta-rule state; per-KV-head decay
half-lives {2048, 45255, 1e6} tokens plus one archival head, beta = sigmoid(N(0,1)), gamma = sigmoid(N(0,1)); the
memory branch receives writes from token 2052 on. Inputs are resident in HBM before the timed region. value =
tokens/s of the whole call (memory-branch projections and gates, delta rule, window attention with the gamma mix,
ring and state write-back).

roofline: the dominant kernel, the window attention (window_fa_kernel), priced on its algorithmic work
4 D FLOP per visible (query, key) pair and query head, over its average launch duration measured with HIP events
on the launch stream with the layer's own arguments.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra] [--only LEG]
Prints ONE JSON line. Only one GPU is supported (--gpus > 1 exits with a message).
"""
import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

import torch
import torch.nn.functional as F

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "Bifrost-layer prefill tokens/s @32K; decode µs/step @B=64; % of MFMA/HBM roofline"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
C = 64


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def make_inputs(T, H, D, dev, seed=0):
    gen = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(T, H, D, device=dev, generator=gen).bfloat16()
    k = F.normalize(torch.randn(T, H, D, device=dev, generator=gen), dim=-1).bfloat16()
    v = torch.randn(T, H, D, device=dev, generator=gen).bfloat16()
    beta = torch.sigmoid(torch.randn(T, H, device=dev, generator=gen))
    g = -torch.rand(T, H, device=dev, generator=gen) * 1e-3
    return q, k, v, g, beta


def gdn_kernel_flops(T, G, R, D, L):
    """Algorithmic FLOPs of one launch of each kernel of bf_gdn_fwd for one sequence of T tokens, G KV heads, R query
    heads per KV head, segments of L chunks (C = 64). Per chunk and KV head:
      prep     2C^2D (K K^T) + R 2C^2D (q K^T) + C^3/3 (unit-triangular inverse)
      summary  the chunk map on the 2D columns [N | Phi]: K S and K^T v_new 2 * 2C(D)(2D), T' y 2C^2(2D), T' V 2C^2D
               = 8CD^2 + 6C^2D, for the chunks of every segment but the last
      output   K S, K^T v_new 4CD^2, T'(V - e^g K S) 4C^2D, and per query head q S 2CD^2 + attn v_new 2C^2D
    combine    per segment step and KV head: Psi X, 2D^3 (the split-bf16 second pass is not counted)."""
    n = (T + C - 1) // C
    nseg = (n + L - 1) // L
    n_sum = n - ((n - 1) % L + 1)                  # chunks outside the last segment
    return {
        "prep": n * G * ((1 + R) * 2 * C * C * D + C ** 3 / 3),
        "summary": n_sum * G * (8 * C * D * D + 6 * C * C * D),
        "combine": max(nseg - 1, 0) * G * 2 * D ** 3,
        "output": n * G * (4 * C * D * D + 4 * C * C * D + R * (2 * C * D * D + 2 * C * C * D)),
    }


def reference_flops(T, H, D):
    """FLOPs of the reference's chunked algorithm (kernels.py:94-129) per head: T (10CD + 6D^2)."""
    return T * H * (10 * C * D + 6 * D * D)


def gdn_bytes(T, H, D):
    """Algorithmic HBM bytes of the whole operator: bf16 q, k, v in; fp32 g, beta in; fp32 o and state out."""
    return T * H * D * 2 * 3 + T * H * 4 * 2 + T * H * D * 4 + H * D * D * 4


def traffic_from_profile(kernel: str):
    """HBM bytes per launch of `kernel` measured by the rocprofv3 FETCH_SIZE / WRITE_SIZE runs (profiles/)."""
    p = ROOT / "profiles" / "traffic.json"
    try:
        return json.loads(p.read_text()).get(kernel)
    except (OSError, ValueError):
        return None


PHASES = ("prep", "summary", "combine", "output")


def run_gdn(steps, warmup, dev, segment_chunks=0):
    """Headline workload. The timed region is K steps of one bf_gdn_fwd call each (all four phases: PREP, SUMMARY,
    COMBINE, OUTPUT, launched back to back by the library), as a caller runs it. A second pass over K steps runs the
    phases as separate calls with HIP events between them (on the stream the kernels are launched on) for the
    per-kernel times of the roofline; the events between kernels cost a few microseconds each, so that pass is not
    the step time."""
    from heimdall_amd import _lib
    from heimdall_amd._device import gdn_forward, workspace

    T, H, D = 32768, 4, 256
    q, k, v, g, beta = make_inputs(T, H, D, dev)
    o = torch.empty(T, H, D, dtype=torch.float32, device=dev)
    s = torch.empty(1, H, D, D, dtype=torch.float32, device=dev)
    lib = _lib.load()
    L = segment_chunks if segment_chunks > 0 else lib.bf_gdn_segment_chunks(T, 1, H, 1, D)
    nbytes = _lib.ctypes.c_size_t(0)
    _lib.check(lib.bf_gdn_workspace_size(T, 1, H, 1, D, _lib.DTYPE_BF16, L, _lib.ctypes.byref(nbytes)),
               "bf_gdn_workspace_size")
    ws = workspace(nbytes.value, dev)
    bits = (_lib.PHASE_PREP, _lib.PHASE_SUMMARY, _lib.PHASE_COMBINE, _lib.PHASE_OUTPUT)

    def phase(p):
        gdn_forward(q, k, v, g, beta, num_seqs=1, out=o, final_state=s, ws=ws, phases=p, segment_chunks=L)

    for _ in range(warmup):
        phase(_lib.PHASE_ALL)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        phase(_lib.PHASE_ALL)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # per-kernel pass
    stream = torch.cuda.current_stream(dev)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(bits) + 1)] for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record(stream)
        for j, p in enumerate(bits):
            phase(p)
            ev[i][j + 1].record(stream)
    torch.cuda.synchronize()
    ms = {name: sum(e[j].elapsed_time(e[j + 1]) for e in ev) / steps for j, name in enumerate(PHASES)}
    return dict(T=T, H=H, D=D, L=L, wall=wall, phase_ms=ms, inputs=(q, k, v, g, beta))


def cpu_baseline(inputs, budget_s=30.0):
    """The oracle (fp32 PyTorch restatement of the reference's chunked delta rule) on the host cores, on the same
    workload (full T=32768) as long as one run fits the budget, else on a prefix."""
    from oracle import gdn

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    q, k, v, g, beta = (z.detach().float().cpu()[None] for z in inputs)
    T = q.shape[1]
    t = time.perf_counter()
    gdn.delta_rule_chunked(q[:, :4096], k[:, :4096], v[:, :4096], g[:, :4096], beta[:, :4096], 64)   # warm-up
    per_4k = (time.perf_counter() - t) * 1.5          # cost grows slightly faster than linearly in T
    n = T
    while n > 4096 and per_4k * n / 4096 > budget_s / 2:
        n //= 2
    times = []
    for _ in range(3):
        t = time.perf_counter()
        gdn.delta_rule_chunked(q[:, :n], k[:, :n], v[:, :n], g[:, :n], beta[:, :n], 64)
        times.append(time.perf_counter() - t)
        if sum(times) > budget_s:
            break
    best = sorted(times)[len(times) // 2]
    return {"value": n / best, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle delta_rule_chunked fp32, T={n} H=4 D=256 (same synthetic inputs), median of "
                      f"{len(times)} run(s), {cpu_model()}"}


def _cpu(value_units: float, fn, unit: str, sample: str) -> dict:
    """Time one call of an oracle function on all host cores: {"value": units per second, ...} ("port" baseline)."""
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    with torch.no_grad():
        t = time.perf_counter()
        fn()
        dt = time.perf_counter() - t
    return {"value": value_units / dt, "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{sample}, one run, {cpu_model()}"}


def _oracle_layer(H, G, D, d, W, S):
    import types
    from oracle import layer as ol
    m = types.SimpleNamespace(c=ol.Cfg(H, G, D, d))
    ol.convert_params(m, W, S, 1)
    return ol, m


def cpu_decode(B=8):
    """The oracle's student decode step (fp32, memory branch and mix included) for B = 8 of the decode leg's 64
    sequences (H=16, G=4, D=256, W=2048 + 4 sinks, position 100000)."""
    H, G, D, W, S, p, d = 16, 4, 256, 2048, 4, 100000, 1024
    ol, m = _oracle_layer(H, G, D, d, W, S)
    rn = lambda *s: torch.randn(*s)
    pos = torch.arange(p - W, p)
    ring_pos = torch.empty(W, dtype=torch.long)
    ring_pos[pos % W] = pos
    cache = dict(ring_k=rn(B, G, W, D), ring_v=rn(B, G, W, D), ring_km=F.normalize(rn(B, W, G, D), dim=-1),
                 ring_g=-torch.rand(B, W, G) * 1e-3, ring_beta=torch.rand(B, W, G), ring_pos=ring_pos,
                 sink_k=rn(B, G, S, D), sink_v=rn(B, G, S, D), S=rn(B, G, D, D) * 0.02)
    x, q, k, v = rn(B, 1, d), rn(B, 1, H, D), rn(B, 1, G, D), rn(B, 1, G, D)
    qr, kr = rn(B, H, 1, D), rn(B, G, 1, D)
    return _cpu(B, lambda: ol.student(m, x, q, k, v, qr, kr, p, cache), "tokens/s",
                f"oracle layer.student decode step fp32, B={B} of 64, H=16 G=4 D=256 W=2048+4")


def cpu_varlen(n=8192):
    """The oracle's per-sequence delta rule (fp32) on two packed sequences of n / 2 tokens, H=32, D=128."""
    from oracle import gdn
    H, D = 32, 128
    q, v = torch.randn(1, n, H, D), torch.randn(1, n, H, D)
    k = F.normalize(torch.randn(1, n, H, D), dim=-1)
    g, beta = -torch.rand(1, n, H) * 5e-3, torch.rand(1, n, H)
    cu = torch.tensor([0, n // 2, n])
    return _cpu(n, lambda: gdn.delta_rule_varlen(q, k, v, g, beta, cu), "tokens/s",
                f"oracle gdn.delta_rule_varlen fp32, 2 sequences of {n // 2}, H=32 D=128")


def cpu_gdn_layer(n=4096):
    """The oracle's Gated DeltaNet layer core (conv + norms + gates, delta rule, gated norm; fp32) on n tokens, H=32,
    D=128, conv width 4."""
    from oracle import gdn_layer as og
    H, D, K = 32, 128, 4
    C = 3 * H * D
    z, a, b, zg = torch.randn(1, n, C), torch.randn(1, n, H), torch.randn(1, n, H), torch.randn(1, n, H * D)
    w, A_log, dt, nw = torch.randn(C, K) * 0.5, torch.randn(H) * 0.5 - 2, torch.randn(H), torch.ones(D)
    return _cpu(n, lambda: og.layer_core(z, a, b, zg, w, A_log, dt, nw, H, H, D), "tokens/s",
                f"oracle gdn_layer.layer_core fp32, T={n}, H=32 D=128")


def cpu_teacher_decode(B=1, n=32768):
    """The oracle's teacher decode step with retrieval (block summaries, selection, masked attention; fp64 as the
    oracle computes) for B = 1 of the leg's 64 sequences at cache length 32768."""
    from oracle import teacher as ot
    H, G, D = 16, 4, 256
    ret = dict(k=16, block=64, window=2048, sinks=4)
    qr = torch.randn(B, H, 1, D)
    kr, vt = F.normalize(torch.randn(B, G, n, D), dim=-1), torch.randn(B, G, n, D)
    return _cpu(B, lambda: ot.masked_attention(qr, kr, vt, ot.retrieval_mask(qr, kr, ret)), "tokens/s",
                f"oracle teacher retrieval decode step (fp64), B={B} of 64, H=16 G=4 D=256 n={n}")


def cpu_llama_state(B=2):
    """The oracle's state-row builder for B = 2 of the leg's 64 sequences (G=4, D=256, W=2048, S=4)."""
    from oracle import formats as of
    G, D, W, S, n = 4, 256, 2048, 4, 100000
    pos = torch.arange(n - W, n)
    ring_pos = torch.empty(W, dtype=torch.long)
    ring_pos[pos % W] = pos
    c = dict(ring_k=torch.randn(B, G, W, D), ring_v=torch.randn(B, G, W, D), ring_km=torch.randn(B, W, G, D),
             ring_g=torch.rand(B, W, G), ring_beta=torch.rand(B, W, G), ring_pos=ring_pos,
             sink_k=torch.randn(B, G, S, D), sink_v=torch.randn(B, G, S, D), S=torch.randn(B, G, D, D))
    return _cpu(B, lambda: [of.llama_state_row(c, b, n, W, S) for b in range(B)], "rows/s",
                f"oracle formats.llama_state_row, B={B} of 64 rows, G=4 D=256 W=2048 S=4")


def run_decode(steps, warmup, dev):
    """Decode step, B=64, H=16, G=4, D=256, W=2048 + 4 sinks, bf16 ring, fp32 state ~ N(0, 0.02), at position
    100000 (ring full, memory active): the bf_decode_fwd pass alone, inputs resident."""
    from heimdall_amd import _lib
    from heimdall_amd._device import stream_ptr, workspace

    B, H, G, D, W, S = 64, 16, 4, 256, 2048, 4
    R, p = H // G, 100000
    gen = torch.Generator(device=dev).manual_seed(1)
    rn = lambda *shape: torch.randn(*shape, device=dev, generator=gen)
    ring_k, ring_v = rn(B, G, W, D).bfloat16(), rn(B, G, W, D).bfloat16()
    sink_k, sink_v = rn(B, G, S, D).bfloat16(), rn(B, G, S, D).bfloat16()
    ring_km = F.normalize(rn(B, W, G, D), dim=-1)
    ring_g = -torch.rand(B, W, G, device=dev, generator=gen) * 1e-3
    ring_beta = torch.sigmoid(rn(B, W, G))
    ring_pos = torch.tensor([pp for pp in range(p - W, p)], device=dev, dtype=torch.long)
    ring_pos = ring_pos[torch.argsort(ring_pos % W)].contiguous()
    state = rn(B, G, D, D) * 0.02
    qr = F.normalize(rn(B, H, D), dim=-1).bfloat16()
    qm = F.normalize(rn(B, H, D), dim=-1) * D ** -0.5
    kr, v = F.normalize(rn(B, G, D), dim=-1).bfloat16(), rn(B, G, D).bfloat16()
    km = F.normalize(rn(B, G, D), dim=-1)
    g_new = -torch.rand(B, G, device=dev, generator=gen) * 1e-3
    b_new = torch.sigmoid(rn(B, G))
    z = rn(B, H)
    mix_lse, mem_scale = torch.zeros(H, device=dev), torch.full((H,), D ** 0.5, device=dev)
    o = torch.empty(B, H, D, device=dev)
    lib = _lib.load()
    nb = _lib.ctypes.c_size_t(0)
    _lib.check(lib.bf_decode_workspace_size(B, G, R, D, W, _lib.ctypes.byref(nb)), "bf_decode_workspace_size")
    ws = workspace(nb.value, dev)
    st = stream_ptr(dev)
    args = (B, G, R, D, W, S, p, 1, _lib.DTYPE_BF16, _lib.DTYPE_BF16, qr.data_ptr(), qm.data_ptr(), kr.data_ptr(),
            v.data_ptr(), km.data_ptr(), g_new.data_ptr(), b_new.data_ptr(), z.data_ptr(), mix_lse.data_ptr(),
            mem_scale.data_ptr(), sink_k.data_ptr(), sink_v.data_ptr(), S, ring_k.data_ptr(), ring_v.data_ptr(),
            ring_km.data_ptr(), ring_g.data_ptr(), ring_beta.data_ptr(), ring_pos.data_ptr(), state.data_ptr(),
            o.data_ptr(), None, ws.data_ptr(), ws.numel(), st)
    for _ in range(warmup):
        _lib.check(lib.bf_decode_fwd(*args), "bf_decode_fwd")
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(torch.cuda.current_stream(dev))
    rcs = [lib.bf_decode_fwd(*args) for _ in range(steps)]
    e1.record(torch.cuda.current_stream(dev))
    torch.cuda.synchronize()
    for rc in rcs:
        _lib.check(rc, "bf_decode_fwd")
    us = e0.elapsed_time(e1) * 1e3 / steps
    # algorithmic bytes: state read + write, full ring K and V read (W slots) + sinks + new row, queries, outputs
    nbytes = (B * G * D * D * 4 * 2 + B * G * (W + S + 1) * D * 2 * 2 + B * H * D * (2 + 4 + 4)
              + B * G * D * (4 + 2 + 2 + 4))
    gbs = nbytes / (us * 1e-6) / 1e9
    # the same step with the 64 sequences at their own positions (bf_decode_fwd_batch): positions 100000 + 37 b
    # (every sequence's ring full, memory active), per-sequence ring_pos rows and sink blocks
    pos_b = torch.tensor([p + 37 * i for i in range(B)], device=dev, dtype=torch.long)
    rp_b = torch.stack([torch.tensor([pp for pp in range(int(q_) - W, int(q_))], device=dev)[
        torch.argsort(torch.arange(int(q_) - W, int(q_), device=dev) % W)] for q_ in pos_b]).contiguous()
    sk_b, sv_b = sink_k.clone(), sink_v.clone()
    bargs = (B, G, R, D, W, S, pos_b.data_ptr(), 1, _lib.DTYPE_BF16, _lib.DTYPE_BF16, qr.data_ptr(), qm.data_ptr(),
             kr.data_ptr(), v.data_ptr(), km.data_ptr(), g_new.data_ptr(), b_new.data_ptr(), z.data_ptr(),
             mix_lse.data_ptr(), mem_scale.data_ptr(), sk_b.data_ptr(), sv_b.data_ptr(), ring_k.data_ptr(),
             ring_v.data_ptr(), ring_km.data_ptr(), ring_g.data_ptr(), ring_beta.data_ptr(), rp_b.data_ptr(),
             state.data_ptr(), o.data_ptr(), None, ws.data_ptr(), ws.numel(), st)
    for _ in range(warmup):
        _lib.check(lib.bf_decode_fwd_batch(*bargs), "bf_decode_fwd_batch")
    torch.cuda.synchronize()
    e0.record(torch.cuda.current_stream(dev))
    rcs = [lib.bf_decode_fwd_batch(*bargs) for _ in range(steps)]
    e1.record(torch.cuda.current_stream(dev))
    torch.cuda.synchronize()
    for rc in rcs:
        _lib.check(rc, "bf_decode_fwd_batch")
    us_b = e0.elapsed_time(e1) * 1e3 / steps
    gbs_b = nbytes / (us_b * 1e-6) / 1e9
    return {"workload": "decode B=64 H=16 G=4 D=256 W=2048+4 bf16 ring, fp32 state", "us_per_step": us,
            "steps": steps, "roofline": {"bound": "hbm", "kernel": "decode_main_kernel+decode_tail_kernel",
                                         "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                         "frac": gbs / HBM_PEAK_GBS, "bytes_per_step": nbytes},
            "mixed_positions": {"workload": "the same step, the 64 sequences at positions 100000 + 37 b "
                                            "(bf_decode_fwd_batch, per-sequence ring_pos and sinks)",
                                "us_per_step": us_b, "GBs": gbs_b, "frac": gbs_b / HBM_PEAK_GBS}}


def run_varlen(steps, warmup, dev):
    """Native Gated DeltaNet core on packed variable-length input: 4 sequences {8192, 16384, 24576, 16384} via
    cu_seqlens, H=32, D=128, bf16 q/k/v (k L2-normalised, q unscaled), g ~ U[-5e-3, 0], beta = sigmoid(N(0,1)), zero
    initial states, final states returned: kernels.delta_rule_varlen timed with HIP events on the launch stream."""
    from heimdall_amd import kernels

    lens = (8192, 16384, 24576, 16384)
    H, D = 32, 128
    N = sum(lens)
    cu = torch.tensor([0, 8192, 24576, 49152, 65536], dtype=torch.int32, device=dev)
    gen = torch.Generator(device=dev).manual_seed(4)
    q = torch.randn(1, N, H, D, device=dev, generator=gen).bfloat16()
    k = F.normalize(torch.randn(1, N, H, D, device=dev, generator=gen), dim=-1).bfloat16()
    v = torch.randn(1, N, H, D, device=dev, generator=gen).bfloat16()
    beta = torch.sigmoid(torch.randn(1, N, H, device=dev, generator=gen))
    g = -torch.rand(1, N, H, device=dev, generator=gen) * 5e-3
    with torch.no_grad():
        for _ in range(warmup):
            kernels.delta_rule_varlen(q, k, v, g, beta, cu)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            kernels.delta_rule_varlen(q, k, v, g, beta, cu)
        e1.record(stream)
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = reference_flops(N, H, D)
    nbytes = gdn_bytes(N, H, D) - H * D * D * 4 + len(lens) * H * D * D * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": "varlen gated delta rule, 4 seqs {8192,16384,24576,16384}, H=32, D=128, bf16",
            "ms_per_step": ms, "tokens_per_s": N / (ms * 1e-3), "steps": steps,
            "tflops_reference": flops / (ms * 1e-3) / 1e12, "GBs": gbs,
            "roofline": {"bound": "hbm", "kernel": "bf_gdn_fwd varlen (prep, summary, combine, output)",
                         "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                         "algorithmic_bytes": nbytes}}


def run_gdn_layer(steps, warmup, dev):
    """The native Gated DeltaNet layer between its frozen projections on configuration 4's packed input (4 sequences
    {8192, 16384, 24576, 16384}, H = 32 key and value heads, D = 128, conv width 4, bf16): z = in_proj_qkv(x),
    a, b, zg synthetic (the projections are PyTorch matrix products outside the measured core). One step =
    bf_gdn_conv_inputs -> bf_gdn_fwd_gated (the varlen delta rule with the GatedNorm applied to its output rows),
    with HIP events between the two on the launch stream. The conv pass is priced against HBM by its algorithmic
    bytes (each tensor read or written once)."""
    from heimdall_amd import gdn_layer as gl
    from heimdall_amd._device import gdn_forward

    lens = (8192, 16384, 24576, 16384)
    hk = hv = 32
    D, K = 128, 4
    N = sum(lens)
    C = (2 * hk + hv) * D
    cu = torch.tensor([0, 8192, 24576, 49152, 65536], dtype=torch.int32, device=dev)
    torch.manual_seed(5)
    m = gl.GatedDeltaNet(gl.GdnLayerConfig(d=64, lin_hk=hk, lin_hv=hv, lin_dk=D, lin_dv=D, conv_k=K))
    with torch.no_grad():
        m.conv1d.weight.normal_(0, 0.5)
        m.A_log.uniform_(-6, -2)
        m.dt_bias.normal_()
    m = m.to(dev)
    gen = torch.Generator(device=dev).manual_seed(6)
    z = torch.randn(N, C, device=dev, generator=gen).bfloat16()
    a = torch.randn(N, hv, device=dev, generator=gen)
    b = torch.randn(N, hv, device=dev, generator=gen)
    zg = torch.randn(N, hv * D, device=dev, generator=gen).bfloat16()
    w = m.conv1d.weight[:, 0].detach()

    def step(ev=None):
        q, k, v, g, beta = gl.conv_inputs(z, w, None, a, b, m.A_log.detach(), m.dt_bias.detach(), hk, hv, D,
                                          cu_seqlens=cu)
        if ev:
            ev[1].record(stream)
        out, s = gdn_forward(q, k, v, g, beta, num_seqs=len(lens), cu_seqlens=cu,
                             gated_norm=(zg.view(N, hv, D), m.norm.weight.detach(), m.norm.eps))
        return out

    stream = torch.cuda.current_stream(dev)
    with torch.no_grad():
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
        for ev in evs:
            ev[0].record(stream)
            step(ev)
            ev[2].record(stream)
        torch.cuda.synchronize()
    parts = [sum(e[j].elapsed_time(e[j + 1]) for e in evs) / steps for j in range(2)]
    ms = sum(parts)
    conv_bytes = N * (C * 2 + 2 * hv * 4 + 3 * hv * D * 2 + 2 * hv * 4) + C * K * 4
    gb = lambda nbytes, t: nbytes / (t * 1e-3) / 1e9
    return {"workload": "native Gated DeltaNet layer core, 4 packed seqs {8192,16384,24576,16384}, H=32, D=128, "
                        "conv 4, bf16",
            "ms_per_step": ms, "tokens_per_s": N / (ms * 1e-3), "steps": steps,
            "ms": {"conv_inputs": parts[0], "delta_rule_gated_norm": parts[1]},
            "conv_inputs_roofline": {"bound": "hbm", "achieved": gb(conv_bytes, parts[0]), "peak": HBM_PEAK_GBS,
                                     "unit": "GB/s", "frac": gb(conv_bytes, parts[0]) / HBM_PEAK_GBS,
                                     "bytes": conv_bytes}}


def run_teacher(steps, warmup, dev, T=32768):
    """The conversion teacher's causal GQA attention (motor.blockwise_attention, Heimdall/heimdall/motor.py:41-67) on
    the layer's shapes (B=1, H=24, G=4, D=256, bf16, fp32 output): bf_window_fwd with W = T and no sinks, timed with
    HIP events. Algorithmic work: 4 D FLOP per (query, key <= query) pair and query head."""
    from heimdall_amd import motor

    B, H, G, D = 1, 24, 4, 256
    gen = torch.Generator(device=dev).manual_seed(7)
    qr = F.normalize(torch.randn(B, H, T, D, device=dev, generator=gen), dim=-1).bfloat16()
    kr = F.normalize(torch.randn(B, G, T, D, device=dev, generator=gen), dim=-1).bfloat16()
    vt = torch.randn(B, G, T, D, device=dev, generator=gen).bfloat16()
    with torch.no_grad():
        for _ in range(warmup):
            motor.blockwise_attention(qr, kr, vt)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            motor.blockwise_attention(qr, kr, vt)
        e1.record(stream)
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = 4 * D * H * T * (T + 1) // 2
    tf = flops / (ms * 1e-3) / 1e12
    return {"workload": f"teacher causal attention B=1 T={T} H=24 G=4 D=256 bf16", "ms_per_step": ms,
            "tokens_per_s": T / (ms * 1e-3), "steps": steps, "flops": flops,
            "roofline": {"bound": "mfma", "achieved": tf, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": tf / BF16_PEAK_TFLOPS}}


def run_teacher_decode(steps, warmup, dev, retrieval=True, n=32768):
    """One decode step of a kept full-attention layer over a KV cache of n = 32768 positions (B=64, H=16, G=4, D=256,
    bf16): the ``_teacher`` drop-in (heimdall_amd.teacher.teacher, Heimdall/heimdall/hibrit.py:275-290) appending the
    new key / value and attending, with retrieval (k=16 blocks of 64, window 2048, 4 sinks: set_retrieval's defaults,
    hibrit.py:292) or over the whole cache. Timed with HIP events over whole steps (every launch of the step).
    Algorithmic bytes: the attended K and V rows (bf16) plus, with retrieval, the block summaries read by the
    selection (min and max, bf16 like the keys, D each per candidate block)."""
    from heimdall_amd.teacher import set_retrieval, teacher

    B, H, G, D = 64, 16, 4, 256
    S, L, W, K = 4, 64, 2048, 16
    cap = n + steps + warmup + 64
    gen = torch.Generator(device=dev).manual_seed(11)
    kb = F.normalize(torch.randn(B, G, cap, D, device=dev, generator=gen), dim=-1).bfloat16()
    vb = torch.randn(B, G, cap, D, device=dev, generator=gen).bfloat16()
    cache = {"k_buf": kb, "v_buf": vb, "k": kb[:, :, :n], "v": vb[:, :, :n]}
    q = F.normalize(torch.randn(B, H, 1, D, device=dev, generator=gen), dim=-1).bfloat16()
    k1 = F.normalize(torch.randn(B, G, 1, D, device=dev, generator=gen), dim=-1).bfloat16()
    v1 = torch.randn(B, 1, G, D, device=dev, generator=gen).bfloat16()

    class _Layer:
        retrieval = None
    m = _Layer()
    if retrieval:
        set_retrieval(m, k=K, block=L, window=W, sinks=S)
    with torch.no_grad():
        for _ in range(warmup):
            teacher(m, q, k1, v1, cache)
        torch.cuda.synchronize()
        n0 = cache["k"].shape[2]
        stream = torch.cuda.current_stream(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            teacher(m, q, k1, v1, cache)
        e1.record(stream)
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    nm = n0 + steps // 2                                    # mean cache length over the timed steps
    if retrieval:
        nb = (nm - S) // L
        nc = (nm - 1 - W + 1 - S) // L
        keys = S + K * L + (nm - (S + nc * L))
        nbytes = B * G * (keys * D * 2 * 2 + nc * D * 2 * 2)     # summaries are bf16 like the keys
    else:
        keys = nm
        nbytes = B * G * keys * D * 2 * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": f"teacher decode B={B} H={H} G={G} D={D} n={n} bf16 "
                        + (f"retrieval k={K} block={L} window={W} sinks={S}" if retrieval else "full attention"),
            "ms_per_step": ms, "us_per_step": ms * 1e3, "tokens_per_s": B / (ms * 1e-3), "steps": steps,
            "attended_keys": keys, "algorithmic_bytes": nbytes,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS}}


FP32_PEAK_TFLOPS = 157.3      # MI355X dense fp32 MFMA, TFLOP/s


def gdn_bwd_flops(T, G, R, D, C=64):
    """FLOPs of the products bf_gdn_bwd computes (per chunk and KV head: (18 + 10R) C^2 D + (14 + 4R) C D^2 + 4 C^3;
    the masked triangular products counted whole)."""
    n = -(-T // C)
    return n * G * ((18 + 10 * R) * C * C * D + (14 + 4 * R) * C * D * D + 4 * C ** 3)


def run_gdn_bwd(steps, warmup, dev, T=8192, cpu=False):
    """The conversion training's delta-rule backward on one time segment (motor.seq_loss with --parca 8192, the
    layer's head geometry G=4 KV heads x R=6 query heads, D=256, fp32 as the reference trains): bf_gdn_bwd alone
    (inputs, output gradient and final-state gradient resident), timed with HIP events; plus the whole
    forward + backward through motor.delta_rule_gqa's autograd."""
    from heimdall_amd import _lib, motor
    from heimdall_amd._device import stream_ptr

    B, G, R, D = 1, 4, 6, 256
    gen = torch.Generator(device=dev).manual_seed(21)
    rn = lambda *s: torch.randn(*s, device=dev, generator=gen)
    q = rn(B, T, G, R, D) * D ** -0.5
    k = F.normalize(rn(B, T, G, D), dim=-1)
    v = rn(B, T, G, D)
    g = -torch.rand(B, T, G, device=dev, generator=gen) * 0.05
    beta = torch.sigmoid(rn(B, T, G))
    s0 = rn(B, G, D, D) * 0.02
    do, dsf = rn(B, T, G, R, D), rn(B, G, D, D) * 0.02
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dg, db, ds0 = torch.empty_like(g), torch.empty_like(beta), torch.empty_like(s0)
    lib = _lib.load()
    nbytes = _lib.ctypes.c_size_t(0)
    _lib.check(lib.bf_gdn_bwd_workspace_size(B, T, G, R, D, _lib.ctypes.byref(nbytes)), "bf_gdn_bwd_workspace_size")
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=dev)

    def bwd():
        _lib.check(lib.bf_gdn_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
                                  s0.data_ptr(), 1.0, do.data_ptr(), dsf.data_ptr(), B, T, G, R, D, dq.data_ptr(),
                                  dk.data_ptr(), dv.data_ptr(), dg.data_ptr(), db.data_ptr(), ds0.data_ptr(),
                                  ws.data_ptr(), nbytes.value, stream_ptr(dev)), "bf_gdn_bwd")

    def fwd_bwd():
        xs = [x.requires_grad_(True) for x in (q.clone(), k.clone(), v.clone(), g.clone(), beta.clone())]
        st = s0.clone().requires_grad_(True)
        o, s = motor.delta_rule_gqa(*xs, 64, st)
        torch.autograd.grad((o, s), xs + [st], (do, dsf))

    stream = torch.cuda.current_stream(dev)
    res = {}
    for name, fn, n in (("bwd", bwd, steps), ("fwd_bwd", fwd_bwd, max(1, steps // 2))):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        res[name] = e0.elapsed_time(e1) / n
    fl = gdn_bwd_flops(T, G, R, D)
    tf = fl / (res["bwd"] * 1e-3) / 1e12
    out = {"workload": f"delta-rule backward B=1 T={T} G={G} R={R} D={D} fp32 (one training segment)",
           "ms_per_step": res["bwd"], "fwd_bwd_ms": res["fwd_bwd"], "tokens_per_s": T / (res["bwd"] * 1e-3),
           "steps": steps, "flops": fl, "workspace_bytes": nbytes.value,
           "roofline": {"bound": "mfma", "achieved": tf, "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": tf / FP32_PEAK_TFLOPS}}
    host = [x.cpu() for x in (q, k, v, g, beta, do, s0, dsf)]

    def cpu_run():
        # the oracle's gradients (autograd of the restated reference, fp32) on the host, on the same segment
        from oracle import gdn as ogdn
        torch.set_num_threads(len(os.sched_getaffinity(0)))
        t0 = time.perf_counter()
        ogdn.delta_rule_gqa_grads(*host[:5], host[6], host[5], host[7], dtype=torch.float32)
        dt = time.perf_counter() - t0
        return {"value": T / dt, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
                "sample": f"oracle delta_rule_gqa_grads fp32 (autograd), T={T} G={G} R={R} D={D}, "
                          f"one run, {cpu_model()}"}
    if cpu == "later":
        return out, cpu_run
    if cpu:
        out["cpu_baseline"] = cpu_run()
    return out


def run_llama_state(steps, warmup, dev):
    """The llama.cpp state-row formats at the decode geometry (B=64 sequences, G=4, D=256, W=2048, 4 sinks, bf16 ring,
    position 100000): bf_llama_state_pack and bf_llama_state_unpack, each timed with HIP events. Algorithmic bytes:
    pack reads the cache (ring k, v bf16; k_mem, g, beta, state f32) and writes the rows (43.7 MB per sequence);
    unpack reads the rows' region and delta block and writes the cache."""
    from heimdall_amd import formats

    B, G, D, W, S, n = 64, 4, 256, 2048, 4, 100000
    gen = torch.Generator(device=dev).manual_seed(31)
    rn = lambda *s: torch.randn(*s, device=dev, generator=gen)
    c = dict(ring_k=rn(B, G, W, D).bfloat16(), ring_v=rn(B, G, W, D).bfloat16(), ring_km=rn(B, W, G, D),
             ring_g=-torch.rand(B, W, G, device=dev, generator=gen), ring_beta=torch.rand(B, W, G, device=dev,
                                                                                       generator=gen),
             ring_pos=torch.empty(W, dtype=torch.long, device=dev), S=rn(B, G, D, D) * 0.02,
             sink_k=rn(B, G, S, D).bfloat16(), sink_v=rn(B, G, S, D).bfloat16())
    pos = torch.arange(n - W, n, device=dev)
    c["ring_pos"][pos % W] = pos
    cache_bytes = sum(t.numel() * t.element_size() for t in c.values())
    row_bytes = B * formats.llama_state_floats(G, D, W, S) * 4
    LR, C_ = (S + W + 2 + 31) // 32 * 32, 3 * G * D + 2 * G
    read_back = B * (LR * C_ + D * D * G) * 4                # unpack reads the region and the delta, not the planes
    stream = torch.cuda.current_stream(dev)
    rows = formats.pack_llama_state(c, n, W, S)
    res = {}
    for name, fn in (("pack", lambda: formats.pack_llama_state(c, n, W, S)),
                     ("unpack", lambda: formats.unpack_llama_state(rows, n, W, S, G, D, torch.bfloat16))):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        nbytes = cache_bytes + (row_bytes if name == "pack" else read_back)
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"ms": ms, "bytes": nbytes, "GBs": gbs, "frac": gbs / HBM_PEAK_GBS}
    return {"workload": f"llama.cpp state rows B={B} G={G} D={D} W={W} S={S} bf16 ring",
            "pack": res["pack"], "unpack": res["unpack"], "ms_per_step": res["pack"]["ms"] + res["unpack"]["ms"],
            "roofline": {"bound": "hbm", "achieved": res["pack"]["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": res["pack"]["frac"], "kernel": "bf_llama_state_pack (region, V plane, delta kernels)"}}


LAYER_GEOM = dict(B=1, H=24, G=4, D=256, W=2048, S=4, d=5120)   # d: the target model's hidden size
LIVES = (2048.0, 45255.0, 1e6, None)        # decay half-lives of KV heads 0-2 in tokens; head 3 archival


def window_pairs(T, W, S):
    """Visible (query, key) pairs per head over positions 0..T-1: min(p + 1, W + S) each."""
    return sum(min(p + 1, W + S) for p in range(T))


def layer_flops(T, H, G, D, W, S):
    """Algorithmic work of one layer prefill call from an empty cache (T tokens): the window, 4 D FLOP per visible
    (query, key) pair and query head; the memory branch in GQA form (chunked, C = 64), G (6 C D + 4 D^2) + H (4 C D +
    2 D^2) FLOP per token; the D x D projections of the memory inputs, (H + G) 2 D^2 FLOP per token."""
    win = 4 * D * window_pairs(T, W, S) * H
    mem = T * (G * (6 * C * D + 4 * D * D) + H * (4 * C * D + 2 * D * D))
    proj = T * (H + G) * 2 * D * D
    return {"window": win, "memory": mem, "projections": proj, "total": win + mem + proj}


def layer_core(H, G, D, W, S, lives, dev, d=None):
    """A converted core whose gates reproduce the workload's distributions through its own parameters: x [.., d] with
    columns [z_beta (G) | z_gamma (H) | the rest]; ab selects z_beta for the write strengths (the decay logits are 0),
    mix selects z_gamma (mix_lse = 0), so beta = sigmoid(z_beta) and gamma = sigmoid(z_gamma), with zero weights on
    the other d - G - H columns (the projections still read all d of them); fq = fk = I; mem_scale = sqrt(D);
    constant log-decay -ln2 / life per KV head (decay_mask 0 where life is None: the archival head)."""
    import math
    from heimdall_amd import hibrit
    m = hibrit.BifrostCore(hibrit.CoreConfig(H, G, D, d if d else G + H))
    m.convert(W, S, 0)
    with torch.no_grad():
        m.ab.weight.zero_()
        m.ab.bias.zero_()
        m.ab.weight[G:, :G] = torch.eye(G)
        m.mix.weight.zero_()
        m.mix.bias.zero_()
        m.mix.weight[:, G:G + H] = torch.eye(H)
        sp = F.softplus(m.dt_bias)
        for h, life in enumerate(lives):
            if life is not None:
                m.A_log[h] = math.log(math.log(2.0) / life) - math.log(sp[h].item())
        m.decay_mask.copy_(torch.tensor([0.0 if life is None else 1.0 for life in lives]))
    return m.to(dev)


def layer_inputs(B, T, H, G, D, dev, seed=2, d=None):
    """q, k ~ N(0,1) L2-normalised per head, v ~ N(0,1) (bf16); x ~ N(0,1) [B, T, d] in bf16, whose first G + H
    columns are z_beta, z_gamma (d = G + H without the rest, fp32, when d is None); qr = q, kr = k (the window reads
    the same unit vectors; no rotary part)."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    rn = lambda *shape: torch.randn(*shape, device=dev, generator=gen)
    q = F.normalize(rn(B, T, H, D), dim=-1).bfloat16()
    k = F.normalize(rn(B, T, G, D), dim=-1).bfloat16()
    v = rn(B, T, G, D).bfloat16()
    x = rn(B, T, d).bfloat16() if d else torch.cat((rn(B, T, G), rn(B, T, H)), -1)
    return x, q, k, v, q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous()


def time_window_in_layer(m, args, steps, warmup, dev, start=0, cache=None):
    """The window kernel with the arguments the layer call gives it (bf16 operands with their layer strides, the
    first S tokens as sinks, the ring, the gamma mix against a bf16 memory read, fp32 output): the average launch
    duration over `steps` launches, HIP events on the launch stream. From an empty cache (start 0) the ring is empty;
    otherwise `args` is the chunk at position `start` and `cache` the student cache before it (ring and sinks)."""
    from heimdall_amd import _lib
    from heimdall_amd._device import stream_ptr

    x, q, k, v, qr, kr = args
    B, T, H, D = q.shape
    G = k.shape[2]
    W, S = m.window, m.sinks
    if cache is None:
        sk, sv = kr[:, :, :S].contiguous(), v.transpose(1, 2)[:, :, :S].contiguous()
        ring_k = torch.zeros(B, G, W, D, dtype=torch.bfloat16, device=dev)
        ring_v = torch.zeros_like(ring_k)
        ring_pos = torch.full((W,), -1, dtype=torch.long, device=dev)
    else:
        sk, sv = cache["sink_k"].contiguous(), cache["sink_v"].contiguous()
        ring_k, ring_v, ring_pos = cache["ring_k"], cache["ring_v"], cache["ring_pos"]
    gen = torch.Generator(device=dev).manual_seed(9)
    o_mem = torch.randn(B, T, H, D, device=dev, generator=gen).bfloat16()
    from heimdall_amd import hibrit
    z = hibrit._gate_logits(m, x)[1]
    mix_lse, mem_scale = m.mix_lse.detach().float().contiguous(), m.mem_scale.detach().float().contiguous()
    o = torch.empty(B, T, H, D, dtype=torch.float32, device=dev)
    lib = _lib.load()
    st = lambda t_, dims: tuple(int(t_.stride(i)) for i in dims)
    wargs = (B, G, H // G, D, T, W, S, start, _lib.DTYPE_BF16, qr.data_ptr(), *st(qr, (0, 1, 2)), kr.data_ptr(),
             *st(kr, (0, 1, 2)), v.data_ptr(), *st(v, (0, 2, 1)), ring_k.data_ptr(), ring_v.data_ptr(),
             ring_pos.data_ptr(), sk.data_ptr(), sv.data_ptr(), S, 1, o_mem.data_ptr(), _lib.DTYPE_BF16, z.data_ptr(),
             mix_lse.data_ptr(), mem_scale.data_ptr(), o.data_ptr(), _lib.DTYPE_F32, None, stream_ptr(dev))
    for _ in range(warmup):
        _lib.check(lib.bf_window_fwd(*wargs), "bf_window_fwd")
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    rcs = [lib.bf_window_fwd(*wargs) for _ in range(steps)]
    e1.record(stream)
    torch.cuda.synchronize()
    for rc in rcs:
        _lib.check(rc, "bf_window_fwd")
    return e0.elapsed_time(e1) * 1e3 / steps


def run_layer(steps, warmup, dev, T=32768, window_pass=True):
    """The converted layer's prefill over T tokens from an empty cache: heimdall_amd.hibrit.student (the _student
    drop-in), B=1, H=24, G=4, D=256, W=2048 + 4 sinks, bf16 activations, fp32 state. Timed region: `steps` whole
    calls bracketed by device synchronisation. Then the window kernel alone with the layer's arguments for its
    roofline."""
    from heimdall_amd import hibrit

    g_ = LAYER_GEOM
    B, H, G, D, W, S, d = g_["B"], g_["H"], g_["G"], g_["D"], g_["W"], g_["S"], g_["d"]
    m = layer_core(H, G, D, W, S, LIVES, dev, d)
    args = layer_inputs(B, T, H, G, D, dev, d=d)
    with torch.no_grad():
        for _ in range(warmup):
            hibrit.student(m, *args, 0, {})
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            hibrit.student(m, *args, 0, {})
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms = wall * 1e3 / steps
    fl = layer_flops(T, H, G, D, W, S)
    out = {"workload": f"layer prefill B={B} T={T} H={H} G={G} D={D} W={W}+{S} d_model={d} bf16 activations, "
                       f"fp32 state",
           "T": T, "ms_per_step": ms, "tokens_per_s": T / (ms * 1e-3), "steps": steps, "flops": fl,
           "tflops": fl["total"] / (ms * 1e-3) / 1e12,
           "mfma_frac_whole_call": fl["total"] / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS}
    if window_pass:
        with torch.no_grad():
            us = time_window_in_layer(m, args, max(steps, 10), max(warmup // 2, 3), dev)
        tf = fl["window"] / (us * 1e-6) / 1e12
        out["roofline"] = {"bound": "mfma", "kernel": "window_fa_kernel<256>", "achieved": tf,
                           "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": tf / BF16_PEAK_TFLOPS,
                           "traffic": traffic_from_profile("window_fa_kernel"), "launch_us": us,
                           "flops_per_launch": fl["window"]}
    return out, (m, args)


def cpu_layer(m, args, budget_s=40.0):
    """The oracle's student prefill (fp32 PyTorch restatement of _student, all host cores) on the headline's own
    inputs and parameters (copied to the host): the whole 32768-token call when a 4096-token probe predicts it fits
    the budget, else the longest power-of-two prefix that does."""
    import copy
    from oracle import layer as ol

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    mc = copy.deepcopy(m).cpu().float()
    x, q, k, v, qr, kr = (z.detach().float().cpu() for z in args)
    T = x.shape[1]
    sl = lambda n: (x[:, :n], q[:, :n], k[:, :n], v[:, :n], qr[:, :, :n], kr[:, :, :n])
    with torch.no_grad():
        t = time.perf_counter()
        ol.student(mc, *sl(4096), 0, {})
        per_4k = time.perf_counter() - t
        n = T
        while n > 4096 and per_4k * n / 4096 * 1.2 > budget_s:
            n //= 2
        t = time.perf_counter()
        ol.student(mc, *sl(n), 0, {})
        dt = time.perf_counter() - t
    return {"value": n / dt, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle layer.student fp32 prefill from an empty cache on the first {n} of the {T} tokens of "
                      f"the same inputs (H=24 G=4 D=256 W=2048+4), one run after a 4096-token warm-up, "
                      f"{cpu_model()}"}


def run_layer_chunked(dev, T=32768, chunk=2048, reps=3, window_pass=True):
    """The layer driven the way the reference's HybridLM.prefill drives it (Heimdall/heimdall/hibrit.py:718-734): T
    tokens as T / 2048 student calls through the cache, each at its own position (the headline's core and inputs,
    d_model 5120, bf16). Timed: whole prefills (every chunk call) bracketed by device synchronisation, `reps` of them
    after one warm-up. The dominant kernel is timed alone on a chunk in the steady state: 2048 queries at position
    T - 2048 over a full ring, HIP events on the launch stream."""
    from heimdall_amd import hibrit

    g_ = LAYER_GEOM
    B, H, G, D, W, S, d = g_["B"], g_["H"], g_["G"], g_["D"], g_["W"], g_["S"], g_["d"]
    m = layer_core(H, G, D, W, S, LIVES, dev, d)
    args = layer_inputs(B, T, H, G, D, dev, d=d)
    sl = lambda a, e: (args[0][:, a:e], args[1][:, a:e], args[2][:, a:e], args[3][:, a:e], args[4][:, :, a:e],
                       args[5][:, :, a:e])

    def prefill(upto=T):
        cache = {}
        for a in range(0, upto, chunk):
            hibrit.student(m, *sl(a, min(a + chunk, upto)), a, cache)
        return cache

    with torch.no_grad():
        prefill()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            prefill()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / reps
    fl = layer_flops(T, H, G, D, W, S)
    out = {"workload": f"layer prefill as {T // chunk} calls of {chunk} tokens through the cache, B={B} T={T} H={H} "
                       f"G={G} D={D} W={W}+{S} d_model={d} bf16",
           "T": T, "chunk": chunk, "ms_per_prefill": ms, "tokens_per_s": T / (ms * 1e-3), "reps": reps,
           "ms_per_chunk_call": ms / (T // chunk), "flops": fl["total"],
           "mfma_frac_whole_prefill": fl["total"] / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS}
    if window_pass:
        with torch.no_grad():
            p0 = T - chunk
            cache = prefill(p0)
            us = time_window_in_layer(m, sl(p0, T), 20, 3, dev, start=p0, cache=cache)
        wfl = 4 * D * H * chunk * (W + S)
        tf = wfl / (us * 1e-6) / 1e12
        out["roofline"] = {"bound": "mfma", "kernel": "window_fa_kernel<256>, 2048 queries over a full ring",
                           "achieved": tf, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": tf / BF16_PEAK_TFLOPS,
                           "launch_us": us, "flops_per_launch": wfl}
    return out


def run_mtp_verify(dev, P=32768, steps=200, warmup=20):
    """The MTP verification step of the reference's generate (Heimdall/heimdall/hibrit.py:758-771): after a prefill of
    P tokens, the layer's student call on t = 2 tokens (the last token and the draft) at the current position, B = 1,
    each step two positions further (an accepted draft); next to it, the plain decode step t = 1. The headline's core
    (H=24, G=4, D=256, W=2048 + 4, d_model 5120, bf16). Timed with HIP events over `steps` calls; the cache snapshot
    the reference takes before each verify is not included. The step is ~11 small launches from Python, so the
    garbage left by the earlier legs is collected before the timed loops: without that, the loop's own allocations
    triggered collections over ~170 K objects of those legs, 279 instead of 115 us per step."""
    import gc
    from heimdall_amd import hibrit

    g_ = LAYER_GEOM
    B, H, G, D, W, S, d = g_["B"], g_["H"], g_["G"], g_["D"], g_["W"], g_["S"], g_["d"]
    m = layer_core(H, G, D, W, S, LIVES, dev, d)
    n = P + 2 * (steps + warmup) + 2
    args = layer_inputs(B, n, H, G, D, dev, d=d)
    sl = lambda a, e: (args[0][:, a:e], args[1][:, a:e], args[2][:, a:e], args[3][:, a:e], args[4][:, :, a:e],
                       args[5][:, :, a:e])
    stream = torch.cuda.current_stream(dev)
    res = {}
    with torch.no_grad():
        for t in (2, 1):
            cache = {}
            for a in range(0, P, 2048):
                hibrit.student(m, *sl(a, a + 2048), a, cache)
            p = P
            gc.collect()
            for _ in range(warmup):
                hibrit.student(m, *sl(p, p + t), p, cache)
                p += t
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(steps):
                hibrit.student(m, *sl(p, p + t), p, cache)
                p += t
            e1.record(stream)
            torch.cuda.synchronize()
            res[t] = e0.elapsed_time(e1) * 1e3 / steps
    return {"workload": f"MTP verify: layer student call with t=2 at position {P}+, B=1 H={H} G={G} D={D} W={W}+{S} "
                        f"d_model={d} bf16 (decode t=1 beside it)",
            "us_per_verify_step": res[2], "us_per_decode_step": res[1], "steps": steps,
            "tokens_per_s_verify_accepted": 2 / (res[2] * 1e-6)}


def gdn_leg(steps, warmup, dev, cpu):
    """Standalone chunked delta-rule prefill (B=1, T=32768, H=4, D=256, bf16 q/k/v, fp32 state and output), priced
    as an HBM-bound pass over its algorithmic bytes (bf16 q, k, v; fp32 g, beta, o, final state) and, for its
    contraction phases, against the reference algorithm's FLOPs on bf16 MFMA."""
    r = run_gdn(steps, warmup, dev)
    T, H, D = r["T"], r["H"], r["D"]
    ms = r["wall"] * 1e3 / steps
    nbytes, ref_f = gdn_bytes(T, H, D), reference_flops(T, H, D)
    gbs = nbytes / (ms * 1e-3) / 1e9
    pm = r["phase_ms"]
    kf = gdn_kernel_flops(T, H, 1, D, r["L"])
    out = {"workload": f"chunked gated delta rule B=1 T={T} H={H} D={D} bf16 in, fp32 state/output",
           "ms_per_step": ms, "tokens_per_s": T / (ms * 1e-3), "steps": steps, "segment_chunks": r["L"],
           "roofline": {"bound": "hbm", "kernel": "bf_gdn_fwd (prep, summary, combine, output)", "achieved": gbs,
                        "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                        "algorithmic_bytes": nbytes},
           "mfma_reference_flops": {"flops": ref_f, "achieved": ref_f / (ms * 1e-3) / 1e12, "peak": BF16_PEAK_TFLOPS,
                                    "unit": "TFLOP/s", "frac": ref_f / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS},
           "phases_ms": pm, "phased_step_ms": sum(pm.values()),
           "kernel_tflops_own_flops": {k_: kf[k_] / (pm[k_] * 1e-3) / 1e12 for k_ in PHASES},
           "traffic": {k_: traffic_from_profile("gdn_" + k_) for k_ in PHASES}}
    if cpu == "later":
        return out, (lambda: cpu_baseline(r["inputs"]))
    if cpu:
        out["cpu_baseline"] = cpu_baseline(r["inputs"])
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-extra", action="store_true", help="the headline only (no secondary legs)")
    ap.add_argument("--calib", action="store_true",
                    help="first run a 1 GiB read-only pass (torch sum) and a 1 GiB write-only pass (torch fill), the "
                         "known-size kernels that scale the FETCH_SIZE / WRITE_SIZE counters of a profiling run")
    ap.add_argument("--only", choices=("layer", "layer131k", "layer_chunked", "layer_chunked131k", "mtp_verify", "gdn",
                                       "decode", "varlen", "gdn_layer", "teacher", "teacher_decode",
                                       "teacher_decode_full", "gdn_bwd", "llama_state"),
                    default=None,
                    help="run one secondary leg alone and print its JSON object (for per-workload profiling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the Bifrost core needs no inter-GPU exchange; "
              "see the sharding notes in DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calib:
        # counter calibration: 1 GiB read once (a sum) and 1 GiB written once (a fill), four times the 256 MB
        # last-level cache, so neither pass can be served from it; the first two GPU kernels of the run
        buf = torch.empty(256 << 20, dtype=torch.float32, device=dev)
        buf.sum()
        buf.fill_(1.0)
        torch.cuda.synchronize()
        del buf

    if args.only:
        leg = {"layer": lambda: run_layer(args.steps, args.warmup, dev)[0],
               "layer131k": lambda: run_layer(args.steps, args.warmup, dev, T=131072)[0],
               "layer_chunked": lambda: run_layer_chunked(dev),
               "layer_chunked131k": lambda: run_layer_chunked(dev, T=131072, reps=1),
               "mtp_verify": lambda: run_mtp_verify(dev),
               "gdn": lambda: gdn_leg(args.steps, args.warmup, dev, not args.no_cpu),
               "decode": lambda: run_decode(args.steps, args.warmup, dev),
               "varlen": lambda: run_varlen(args.steps, args.warmup, dev),
               "gdn_layer": lambda: run_gdn_layer(args.steps, args.warmup, dev),
               "teacher": lambda: run_teacher(args.steps, args.warmup, dev),
               "teacher_decode": lambda: run_teacher_decode(args.steps, args.warmup, dev),
               "teacher_decode_full": lambda: run_teacher_decode(args.steps, args.warmup, dev, retrieval=False),
               "gdn_bwd": lambda: run_gdn_bwd(args.steps, args.warmup, dev, cpu=not args.no_cpu),
               "llama_state": lambda: run_llama_state(args.steps, args.warmup, dev)}[args.only]
        print(json.dumps(leg()), flush=True)
        return

    r, (m, inputs) = run_layer(args.steps, args.warmup, dev)
    g_ = LAYER_GEOM
    line = {
        "metric": METRIC,
        "value": r["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "layer_prefill", "B": g_["B"], "T": r["T"], "H": g_["H"], "G": g_["G"],
                   "D": g_["D"], "window": g_["W"], "sinks": g_["S"], "chunk": C, "d_model": g_["d"],
                   "inputs": "bf16 activations, fp32 delta-rule state, decay half-lives 2048/45255/1e6 + archival",
                   "parallelism": "single GPU"},
        "roofline": r["roofline"],
        "layer_flops": r["flops"],
        "layer_tflops": r["tflops"],
        "mfma_frac_whole_call": r["mfma_frac_whole_call"],
    }
    if not args.no_extra:
        r131, _ = run_layer(3, 1, dev, T=131072, window_pass=False)
        line["layer_prefill_131k"] = r131
        line["layer_chunked"] = run_layer_chunked(dev)
        line["layer_chunked_131k"] = run_layer_chunked(dev, T=131072, reps=1, window_pass=False)
        line["mtp_verify"] = run_mtp_verify(dev)
        # every GPU leg runs before any CPU baseline: the oracle's host threads must not compete with the launches
        line["gdn_prefill"], cpu_gdn = gdn_leg(args.steps, args.warmup, dev, "later")
        line["decode"] = run_decode(200, 100, dev)
        line["varlen_gdn"] = run_varlen(10, 3, dev)
        line["gdn_layer"] = run_gdn_layer(10, 3, dev)
        line["teacher_decode"] = run_teacher_decode(50, 10, dev)
        line["gdn_bwd"], cpu_bwd = run_gdn_bwd(10, 2, dev, cpu="later")
        line["llama_state"] = run_llama_state(5, 2, dev)
        if not args.no_cpu:
            for leg, fn in (("gdn_prefill", cpu_gdn), ("decode", cpu_decode), ("varlen_gdn", cpu_varlen),
                            ("gdn_layer", cpu_gdn_layer), ("teacher_decode", cpu_teacher_decode),
                            ("gdn_bwd", cpu_bwd), ("llama_state", cpu_llama_state)):
                line[leg]["cpu_baseline"] = fn()
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_layer(m, inputs)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
