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
    """H=24, G=4, D=256, W=2048 + 4 sinks, bf16 activations: a 3000-token prefill then a 1200-token chunk (the
    memory branch becomes active mid-chunk, the window reads across the ring), against the fp32 oracle on the same
    bf16 values."""
    from heimdall_amd import hibrit
    print("layer bf16 H=24 G=4 D=256 W=2048 T=3000+1200", flush=True)
    m = make_core(24, 4, 256, 64, window=2048, sinks=4)
    mg = make_core(24, 4, 256, 64, window=2048, sinks=4).to(dev)
    args = make_inputs(m, 1, 4200, seed=13, dtype=torch.bfloat16)
    argsf = tuple(z.float() for z in args)
    c_ref, c_gpu = {}, {}
    with torch.no_grad():
        for a, e in ((0, 3000), (3000, 4200)):
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
        qm, km, g, beta = hibrit._mem_inputs_bf16(mg, x.to(dev), q.to(dev), k.to(dev), pos.to(dev))
    assert qm.dtype == km.dtype == torch.bfloat16
    for got, ref in ((qm, qm_ref), (km, km_ref), (g, g_ref), (beta, b_ref)):
        assert rel(got, ref) < TOL_BF16, rel(got, ref)
    print(f"  rel qm={rel(qm, qm_ref):.2e} km={rel(km, km_ref):.2e}", flush=True)
    # rows are unit vectors times the scale
    nq = qm.float().norm(dim=-1).cpu()
    assert torch.allclose(nq, torch.full_like(nq, d ** -0.5), rtol=1e-2)
