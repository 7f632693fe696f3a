"""GPU parity of the converted layer's student path (K1 + K2 prefill, K3 decode) against the CPU oracle: full
sequences, chunked/cached runs mixing prefill chunks and single tokens (the split of the reference's
test_chunked_cache_equals_full), the memory-off mode, and a bf16 run at production head geometry.
Tolerances (relative L2): <= 1e-4 for fp32 runs, <= 2e-2 for bf16 runs against the fp32 oracle."""
import pytest
import torch

from oracle import layer as olayer
from test_gpu_decode import compare_caches, make_core, make_inputs, rel, split, to_dev

pytestmark = pytest.mark.gpu

TOL_F32, TOL_BF16 = 1e-4, 2e-2


@pytest.mark.parametrize("memory", [True, False])
def test_full_sequence_fp32(dev, memory):
    from heimdall_amd import hibrit
    print(f"layer fp32 full B=2 H=4 G=2 D=64 W=16 S=2 T=61 memory={memory}", flush=True)
    m = make_core(4, 2, 64, 32, window=16, sinks=2)
    mg = make_core(4, 2, 64, 32, window=16, sinks=2).to(dev)
    args = make_inputs(m, 2, 61, seed=11)
    with torch.no_grad():
        o_ref = olayer.student(m, *args, 0, None, memory)
        o = hibrit.student(mg, *to_dev(args, dev), 0, None, memory)
    assert rel(o, o_ref) < TOL_F32, rel(o, o_ref)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_chunked_cache_equals_oracle_fp32(dev, d):
    """Chunk splits 5,1,13,1,1,9,30,1 (prefill chunks and single tokens across ring boundaries); every chunk's
    output and the final cache match the oracle run with the same splits, and the GPU chunked run matches the GPU
    full-sequence run."""
    from heimdall_amd import hibrit
    print(f"layer fp32 chunked D={d}", flush=True)
    m = make_core(4, 2, d, 32, window=8, sinks=2)
    mg = make_core(4, 2, d, 32, window=8, sinks=2).to(dev)
    args = make_inputs(m, 1, 61, seed=12)
    c_ref, c_gpu, a = {}, {}, 0
    outs, outs_ref = [], []
    with torch.no_grad():
        for n in (5, 1, 13, 1, 1, 9, 30, 1):
            outs_ref.append(olayer.student(m, *split(args, a, a + n), a, c_ref))
            outs.append(hibrit.student(mg, *to_dev(split(args, a, a + n), dev), a, c_gpu))
            assert rel(outs[-1], outs_ref[-1]) < TOL_F32, (a, n, rel(outs[-1], outs_ref[-1]))
            a += n
        full = hibrit.student(mg, *to_dev(args, dev), 0, None)
    compare_caches(c_ref, c_gpu, TOL_F32)
    assert rel(torch.cat(outs, 1), full) < TOL_F32


def test_production_geometry_bf16(dev):
    """H=24, G=4, D=256, W=2048 + 4 sinks, bf16 activations: a 3000-token prefill, a 1200-token chunk (the memory
    branch becomes active mid-chunk, the window reads across the ring), a 2048-token chunk over a full ring, then
    chunks of 2 and 5 tokens (an MTP verification step), against the fp32 oracle on the same bf16 values. The
    window's work items of 128 queries x 1 head are 576, 240, 384, 24 and 24: the first and third leave a last round
    of at most 16 items on each XCD, which run as two key halves each (merged afterwards), the second does not, and
    the last two run each item as 5 key parts of ~7 of the 35 key blocks."""
    from heimdall_amd import hibrit
    print("layer bf16 H=24 G=4 D=256 W=2048 T=3000+1200+2048+2+5", flush=True)
    m = make_core(24, 4, 256, 64, window=2048, sinks=4)
    mg = make_core(24, 4, 256, 64, window=2048, sinks=4).to(dev)
    args = make_inputs(m, 1, 6255, seed=13, dtype=torch.bfloat16)
    argsf = tuple(z.float() for z in args)
    c_ref, c_gpu = {}, {}
    with torch.no_grad():
        for a, e in ((0, 3000), (3000, 4200), (4200, 6248), (6248, 6250), (6250, 6255)):
            o_ref = olayer.student(m, *split(argsf, a, e), a, c_ref)
            o = hibrit.student(mg, *to_dev(split(args, a, e), dev), a, c_gpu)
            print(f"  chunk {a}:{e} rel err {rel(o, o_ref):.2e}", flush=True)
            assert rel(o, o_ref) < TOL_BF16
    assert rel(c_gpu["S"], c_ref["S"]) < TOL_BF16


@pytest.mark.parametrize("d", [64, 128, 256])
def test_mem_inputs_bf16_fused_projection(dev, d):
    """bf_mem_project (qm, km of _mem_inputs for bf16 activations) against the oracle's fp32 mem_inputs with trained-
    like projections (identity + noise) on the same bf16 values; strided q (a [B, T, H, D] view of a wider tensor),
    B = 2, a token count that is not a multiple of the 64-token tile."""
    from heimdall_amd import hibrit
    print(f"mem_inputs bf16 fused projection D={d}", flush=True)
    m = make_core(6, 2, d, 32, window=16, sinks=2)
    mg = make_core(6, 2, d, 32, window=16, sinks=2).to(dev)
    b, t = 2, 157
    gen = torch.Generator().manual_seed(21)
    x = torch.randn(b, t, 32, generator=gen)
    qw = torch.randn(b, t, 8, d, generator=gen).bfloat16()
    q = qw[:, :, 1:7]                                      # strided head view
    k = torch.randn(b, t, 2, d, generator=gen).bfloat16()
    pos = torch.arange(t)
    qm_ref, km_ref, g_ref, b_ref = olayer.mem_inputs(m, x, q.float(), k.float(), pos)
    with torch.no_grad():
        ab, _ = hibrit._gate_logits(mg, x.to(dev))
        qm, km, g, beta = hibrit._mem_inputs_bf16(mg, ab, q.to(dev), k.to(dev), 0)
    assert qm.dtype == km.dtype == torch.bfloat16
    for got, ref in ((qm, qm_ref), (km, km_ref), (g, g_ref), (beta, b_ref)):
        assert rel(got, ref) < TOL_BF16, rel(got, ref)
    print(f"  rel qm={rel(qm, qm_ref):.2e} km={rel(km, km_ref):.2e}", flush=True)
    # rows are unit vectors times the scale
    nq = qm.float().norm(dim=-1).cpu()
    assert torch.allclose(nq, torch.full_like(nq, d ** -0.5), rtol=1e-2)


def test_mem_gates_and_projection_cache(dev):
    """bf_mem_gates (the gates of _mem_inputs for bf16 activations) against the oracle's fp32 gates for B = 2
    sequences starting at position 1 with 2 sinks (beta is zero at position 1), relative error <= 1e-5; then changes
    of fq reach the next projection: an in-place step on the Parameter (as an optimizer step makes) and a write
    through ``.data`` (as the reference's apply_conversion makes, hibrit.py:798), which leaves no version bump."""
    from heimdall_amd import hibrit
    print("mem_inputs bf16 gates and F^T cache, D=64", flush=True)
    m = make_core(6, 2, 64, 32, window=16, sinks=2)
    mg = make_core(6, 2, 64, 32, window=16, sinks=2).to(dev)
    with torch.no_grad():                                  # non-trivial gates: trained-like ab, one archival head
        gen0 = torch.Generator().manual_seed(5)
        w_ab, b_ab = torch.randn(4, 32, generator=gen0), torch.randn(4, generator=gen0)
        for mm in (m, mg):
            mm.ab.weight.copy_(w_ab)
            mm.ab.bias.copy_(b_ab)
    b, t, start = 2, 70, 1
    gen = torch.Generator().manual_seed(22)
    x = torch.randn(b, t, 32, generator=gen)
    q = torch.randn(b, t, 6, 64, generator=gen).bfloat16()
    k = torch.randn(b, t, 2, 64, generator=gen).bfloat16()
    pos = torch.arange(start, start + t)
    _, _, g_ref, b_ref = olayer.mem_inputs(m, x, q.float(), k.float(), pos)
    with torch.no_grad():
        ab, _ = hibrit._gate_logits(mg, x.to(dev))
        qm0, _, g, beta = hibrit._mem_inputs_bf16(mg, ab, q.to(dev), k.to(dev), start)
    assert rel(g, g_ref) < 1e-5 and rel(beta, b_ref) < 1e-5, (rel(g, g_ref), rel(beta, b_ref))
    assert beta[:, 0].abs().max().item() == 0.0
    noise = torch.randn(m.fq.shape, generator=gen) * 0.3
    with torch.no_grad():
        m.fq.add_(noise)
        mg.fq.add_(noise.to(dev))
        qm1, _, _, _ = hibrit._mem_inputs_bf16(mg, ab, q.to(dev), k.to(dev), start)
    qm_ref, _, _, _ = olayer.mem_inputs(m, x, q.float(), k.float(), pos)
    assert rel(qm1, qm_ref) < TOL_BF16 and rel(qm1, qm0) > 10 * TOL_BF16, (rel(qm1, qm_ref), rel(qm1, qm0))
    new_fq = torch.eye(64).repeat(6, 1, 1) + torch.randn(m.fq.shape, generator=gen) * 0.3
    with torch.no_grad():
        m.fq.data.copy_(new_fq)
        mg.fq.data.copy_(new_fq.to(dev))
        qm2, _, _, _ = hibrit._mem_inputs_bf16(mg, ab, q.to(dev), k.to(dev), start)
    qm_ref2, _, _, _ = olayer.mem_inputs(m, x, q.float(), k.float(), pos)
    assert rel(qm2, qm_ref2) < TOL_BF16 and rel(qm2, qm1) > 10 * TOL_BF16, (rel(qm2, qm_ref2), rel(qm2, qm1))


@pytest.mark.parametrize("b,t,d,n1", [(1, 1000, 5120, 24), (2, 37, 40, 24), (1, 130, 1024, 0), (3, 16, 256, 56),
                                      (1, 1, 5120, 24), (1, 4100, 512, 24), (1, 4200, 1000, 56), (2, 2600, 264, 0)])
def test_gate_project(dev, b, t, d, n1):
    """bf_gate_project (the ab and mix projections of a bf16 chunk in one pass) against fp32 products of the same
    bf16 x: relative error <= 1e-5 per output (W split into bf16 high and low parts); d = 40 ends on a partial
    32-wide step, n1 = 0 has one output, n0 + n1 = 64 is the widest; one token (a decode step). Above 4096 tokens the
    LDS-tiled kernel runs on W split into the workspace: 256-wide steps up to 32 outputs (4100 tokens; 5200 tokens
    with d = 264 ending on a partial step), 128-wide steps for 64 outputs with d = 1000 ending inside a step. A
    strided x view (every other token row of a wider tensor) goes through _gate_logits. Both paths need their
    workspace, and each is run twice and must reproduce its bits."""
    from heimdall_amd import _lib
    from heimdall_amd._device import stream_ptr
    print(f"gate projection B={b} t={t} d={d} n0=8 n1={n1}", flush=True)
    gen = torch.Generator().manual_seed(31 + d)
    x = torch.randn(b * t, d, generator=gen).bfloat16()
    w0, b0 = torch.randn(8, d, generator=gen) * d ** -0.5, torch.randn(8, generator=gen)
    w1, b1 = torch.randn(max(n1, 1), d, generator=gen) * d ** -0.5, torch.randn(max(n1, 1), generator=gen)
    ref0 = x.double() @ w0.double().T + b0.double()
    ref1 = x.double() @ w1.double().T + b1.double()
    xd, w0d, b0d, w1d, b1d = (z.to(dev).contiguous() for z in (x, w0, b0, w1, b1))
    o0 = torch.empty(b * t, 8, device=dev)
    o1 = torch.empty(b * t, max(n1, 1), device=dev)
    lib = _lib.load()
    nb = _lib.ctypes.c_size_t(0)
    assert lib.bf_gate_project_workspace_size(b * t, d, 8 + n1, _lib.ctypes.byref(nb)) == 0
    assert nb.value > 0
    if b * t > 4096:                       # W^T split: 2 ceil(d / 256) sub-steps x 8 KB per 16 outputs
        assert nb.value == 2 * ((d + 255) // 256) * ((8 + n1 + 15) // 16) * 8192
    ws = torch.empty(nb.value, dtype=torch.uint8, device=dev)
    run = lambda: lib.bf_gate_project(xd.data_ptr(), b * t, d, d, w0d.data_ptr(), b0d.data_ptr(), 8, o0.data_ptr(),
                                      w1d.data_ptr() if n1 else None, b1d.data_ptr() if n1 else None, n1,
                                      o1.data_ptr() if n1 else None, ws.data_ptr(), nb.value, stream_ptr(dev))
    assert lib.bf_gate_project(xd.data_ptr(), b * t, d, d, w0d.data_ptr(), b0d.data_ptr(), 8, o0.data_ptr(),
                               w1d.data_ptr() if n1 else None, b1d.data_ptr() if n1 else None, n1,
                               o1.data_ptr() if n1 else None, None, 0, stream_ptr(dev)) != 0   # no workspace
    rc = run()
    assert rc == 0, rc
    first = (o0.clone(), o1.clone())
    assert run() == 0
    assert torch.equal(o0, first[0]) and torch.equal(o1, first[1])
    e0 = rel(o0, ref0)
    assert e0 < 1e-5, e0
    if n1:
        e1 = rel(o1, ref1)
        assert e1 < 1e-5, e1
    # the host helper on a strided view (token stride 2 d): the kernel path, equal to the fp32 torch path
    if d % 8 == 0 and n1 == 24:
        from heimdall_amd import hibrit
        G, H = 4, 24
        core = make_core(H, G, 64, d, window=16, sinks=2)
        with torch.no_grad():
            core.ab.weight.copy_(w0)
            core.ab.bias.copy_(b0)
            core.mix.weight.copy_(w1)
            core.mix.bias.copy_(b1)
        core = core.to(dev)
        wide = torch.randn(b, 2 * t, d, generator=gen).bfloat16().to(dev)
        xv = wide[:, ::2]
        with torch.no_grad():
            ab, z = hibrit._gate_logits(core, xv)
            ab_ref = torch.nn.functional.linear(xv.double(), core.ab.weight.double(), core.ab.bias.double())
            z_ref = torch.nn.functional.linear(xv.double(), core.mix.weight.double(), core.mix.bias.double())
        assert rel(ab, ab_ref) < 1e-5 and rel(z, z_ref) < 1e-5, (rel(ab, ab_ref), rel(z, z_ref))


@pytest.mark.parametrize("b", [1, 3])
def test_fused_prefill_batch_bf16(dev, b):
    """bf_layer_prefill_fwd over B sequences: a prefill from the empty cache past the window (the shifted write
    stream; staged query and output rows when B > 1), a chunk whose stream starts in the ring, a decode token and a
    chunk longer than the window, bf16 activations against the fp32 oracle; the final caches match."""
    from heimdall_amd import hibrit
    print(f"layer bf16 fused prefill B={b} H=6 G=2 D=128 W=16 S=2 chunks 20,7,1,40", flush=True)
    m = make_core(6, 2, 128, 32, window=16, sinks=2)
    mg = make_core(6, 2, 128, 32, window=16, sinks=2).to(dev)
    args = make_inputs(m, b, 68, seed=14, dtype=torch.bfloat16)
    argsf = tuple(z.float() for z in args)
    c_ref, c_gpu, a = {}, {}, 0
    with torch.no_grad():
        for n in (20, 7, 1, 40):
            o_ref = olayer.student(m, *split(argsf, a, a + n), a, c_ref)
            o = hibrit.student(mg, *to_dev(split(args, a, a + n), dev), a, c_gpu)
            print(f"  chunk {a}:{a + n} rel err {rel(o, o_ref):.2e}", flush=True)
            assert rel(o, o_ref) < TOL_BF16
            a += n
    compare_caches(c_ref, c_gpu, TOL_BF16)


def test_fused_prefill_mixed_memory_dtype(dev):
    """fp32 memory inputs (qm, km) with bf16 window inputs: the library converts the memory rows to the compute
    dtype (the query and stream kernels) instead of reading them in place; same result as all-bf16 inputs to
    bf16 rounding."""
    from heimdall_amd import hibrit
    print("layer fused prefill fp32 qm/km with bf16 q/k/v, B=1 H=4 G=2 D=64 W=8", flush=True)
    m = make_core(4, 2, 64, 32, window=8, sinks=2)
    mg = make_core(4, 2, 64, 32, window=8, sinks=2).to(dev)
    x, q, k, v, qr, kr = to_dev(make_inputs(m, 1, 40, seed=15, dtype=torch.bfloat16), dev)
    pos = torch.arange(40, device=dev)
    with torch.no_grad():
        qm, km, g, beta = mg._mem_inputs(x.float(), q.float(), k.float(), pos)
        outs = []
        for mem_dt in (torch.float32, torch.bfloat16):
            st = {}
            st.update(hibrit._new_ring(1, 2, 8, 64, torch.bfloat16, torch.bfloat16, dev))
            o = hibrit._prefill(mg, x, qr, kr, v, qm.to(mem_dt), km.to(mem_dt), g, beta, 0, st, kr[:, :, :2],
                                v.transpose(1, 2)[:, :, :2], True)
            outs.append((o, st["S"]))
    assert rel(outs[0][0], outs[1][0]) < TOL_BF16
    assert rel(outs[0][1], outs[1][1]) < TOL_BF16
