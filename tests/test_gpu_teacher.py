"""GPU parity of the kept full-attention layers' path (``heimdall_amd.teacher``) against ``oracle.teacher``: block
summaries (exact), the retrieval selection (the same block sets), split-K attention over a KV cache with and without
retrieval, and the ``_teacher`` drop-in over prefill / chunked prefill / decode with a growing cache.

Tolerances: relative L2 <= 1e-4 for fp32 runs; <= 2e-2 for bf16 runs against the fp64 oracle on the same
bf16-rounded inputs. Block min / max and the selected block ids are compared exactly."""
import pytest
import torch

from oracle import teacher as ot

pytestmark = pytest.mark.gpu

TOL32, TOL16 = 1e-4, 2e-2


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def tol(dtype):
    return TOL32 if dtype == torch.float32 else TOL16


def cache_tensors(seed, B, G, n, D, dtype, cap=None):
    """k, v [B, G, n, D] as views of [B, G, cap, D] buffers (the layout the teacher keeps)."""
    g = torch.Generator().manual_seed(seed)
    cap = cap or n
    kb = torch.randn(B, G, cap, D, generator=g).to(dtype)
    vb = torch.randn(B, G, cap, D, generator=g).to(dtype)
    return kb, vb


@pytest.mark.parametrize("dtype,D", [(torch.float32, 64), (torch.bfloat16, 128), (torch.bfloat16, 256)])
def test_block_summary_exact_and_incremental(dev, dtype, D):
    from heimdall_amd.teacher import kv_block_summary, summaries_as_blocks, summary_buffers
    B, G, n, S, L = 2, 3, 300, 4, 16
    kb, _ = cache_tensors(1, B, G, n + 37, D, dtype)
    nb = (n - S) // L
    kmin, kmax = summary_buffers(B, G, D, nb + 5, dtype, dev)
    kmin.fill_(7.0)
    kmax.fill_(7.0)
    k = kb.to(dev)
    print(f"summary {dtype} D={D}", flush=True)
    kv_block_summary(k, S, L, 10, nb, kmin, kmax)             # blocks 10 .. nb - 1 only
    lo_b, hi_b = summaries_as_blocks(kmin), summaries_as_blocks(kmax)
    assert (lo_b[:, :, :10] == 7.0).all() and (lo_b[:, :, nb:] == 7.0).all() and (hi_b[:, :, nb:] == 7.0).all()
    kv_block_summary(k, S, L, 0, 10, kmin, kmax)
    lo, hi = ot.block_summary(kb[:, :, :n].float(), S, L)
    lo_b, hi_b = summaries_as_blocks(kmin), summaries_as_blocks(kmax)
    assert torch.equal(lo_b[:, :, :nb].cpu().double(), lo) and torch.equal(hi_b[:, :, :nb].cpu().double(), hi)


@pytest.mark.parametrize("dtype,D,R,T,K", [(torch.float32, 64, 1, 1, 4), (torch.bfloat16, 128, 4, 1, 16),
                                           (torch.bfloat16, 256, 8, 3, 8), (torch.float32, 128, 2, 5, 64)])
def test_select_matches_oracle(dev, dtype, D, R, T, K):
    from heimdall_amd.teacher import kv_block_summary, kv_select, summary_buffers
    B, G, n, S, L, W = 2, 2, 1500, 4, 16, 200
    g = torch.Generator().manual_seed(2)
    kb, _ = cache_tensors(3, B, G, n, D, dtype)
    q = torch.randn(B, T, G * R, D, generator=g).to(dtype)
    nb = (n - S) // L
    kmin, kmax = summary_buffers(B, G, D, nb, dtype, dev)
    kv_block_summary(kb.to(dev), S, L, 0, nb, kmin, kmax)
    ret = dict(k=K, block=L, window=W, sinks=S)
    print(f"select {dtype} D={D} R={R} T={T} K={K}", flush=True)
    sel = kv_select(q.to(dev), n, ret, kmin, kmax).cpu()
    want, nc = ot.select_blocks(q.float().transpose(1, 2), kb.float(), K, L, W, S)   # [B, G, T, nb]
    for b in range(B):
        for i in range(T):
            for gg in range(G):
                ids = sel[b, i, gg]
                got = set(ids[ids >= 0].tolist())
                exp = set(torch.nonzero(want[b, gg, i]).flatten().tolist())
                assert got == exp, (b, i, gg)
                assert (ids >= 0).sum() == min(K, int(nc[i]))


def test_select_fewer_candidates_than_k(dev):
    """Early in a sequence fewer than k blocks lie before the window: the rest of sel is -1."""
    from heimdall_amd.teacher import kv_block_summary, kv_select, summary_buffers
    B, G, D, S, L, W, K = 1, 1, 64, 4, 8, 40, 16
    n = S + W + 5 * L                       # 5 candidates for the last query
    kb, _ = cache_tensors(4, B, G, n, D, torch.float32)
    q = torch.randn(B, 1, 2, D, generator=torch.Generator().manual_seed(5))
    nb = (n - S) // L
    kmin, kmax = summary_buffers(B, G, D, nb, torch.float32, dev)
    kv_block_summary(kb.to(dev), S, L, 0, nb, kmin, kmax)
    sel = kv_select(q.to(dev), n, dict(k=K, block=L, window=W, sinks=S), kmin, kmax).cpu()
    assert sorted(sel[0, 0, 0, :5].tolist()) == [0, 1, 2, 3, 4]
    assert (sel[0, 0, 0, 5:] == -1).all()


@pytest.mark.parametrize("K", [1, 17, 64])
def test_select_ties_and_many_blocks(dev, K):
    """3000 candidate blocks (several per lane of every wave's slice), whose contents repeat with period 7, so equal
    bounds abound: the selection keeps the lower block ids, as the oracle's stable order does."""
    from heimdall_amd.teacher import kv_block_summary, kv_select, summary_buffers
    B, G, R, D, S, L, W = 1, 2, 3, 64, 4, 8, 64
    n = S + 3000 * L + W
    g = torch.Generator().manual_seed(13)
    base = torch.randn(B, G, 7 * L, D, generator=g)
    kb = torch.cat((torch.randn(B, G, S, D, generator=g), base.repeat(1, 1, n // (7 * L) + 1, 1)), 2)[:, :, :n]
    q = torch.randn(B, 1, G * R, D, generator=g)
    nb = (n - S) // L
    kmin, kmax = summary_buffers(B, G, D, nb, torch.float32, dev)
    kv_block_summary(kb.to(dev), S, L, 0, nb, kmin, kmax)
    print(f"select ties K={K} nb={nb}", flush=True)
    sel = kv_select(q.to(dev), n, dict(k=K, block=L, window=W, sinks=S), kmin, kmax).cpu()
    want, nc = ot.select_blocks(q.transpose(1, 2), kb, K, L, W, S)
    for gg in range(G):
        assert sorted(sel[0, 0, gg].tolist()) == torch.nonzero(want[0, gg, 0]).flatten().tolist(), gg


@pytest.mark.parametrize("dtype,D,R,T,n", [(torch.float32, 64, 2, 1, 700), (torch.bfloat16, 128, 4, 1, 3000),
                                           (torch.bfloat16, 256, 8, 4, 1100), (torch.float32, 256, 1, 3, 513),
                                           (torch.bfloat16, 64, 3, 16, 16)])
def test_kv_attention_causal(dev, dtype, D, R, T, n):
    """No retrieval: each of the T trailing queries attends to every key up to its position (several splits)."""
    from heimdall_amd.teacher import kv_attention
    B, G = 2, 2
    kb, vb = cache_tensors(6, B, G, n, D, dtype, cap=n + 64)  # strided views of a larger buffer
    q = torch.randn(B, T, G * R, D, generator=torch.Generator().manual_seed(7)).to(dtype)
    print(f"kv causal {dtype} D={D} R={R} T={T} n={n}", flush=True)
    o = kv_attention(q.to(dev), kb.to(dev), vb.to(dev), n)
    qr = q.float().transpose(1, 2)
    ref = ot.masked_attention(qr, kb[:, :, :n].float(), vb[:, :, :n].float(), ot.teacher_mask(qr, kb[:, :, :n], None))
    assert rel(o, ref) < tol(dtype)


@pytest.mark.parametrize("dtype,D,R,T,K", [(torch.float32, 64, 2, 1, 8), (torch.bfloat16, 128, 4, 1, 16),
                                           (torch.bfloat16, 256, 8, 1, 4), (torch.bfloat16, 128, 2, 6, 0),
                                           (torch.float32, 128, 4, 5, 64)])
def test_kv_attention_retrieval(dev, dtype, D, R, T, K):
    from heimdall_amd.teacher import kv_attention, kv_block_summary, kv_select, summary_buffers
    B, G, n, S, L, W = 2, 2, 2600, 4, 32, 300
    kb, vb = cache_tensors(8, B, G, n, D, dtype)
    q = torch.randn(B, T, G * R, D, generator=torch.Generator().manual_seed(9)).to(dtype)
    ret = dict(k=K, block=L, window=W, sinks=S)
    nb = (n - S) // L
    kmin, kmax = summary_buffers(B, G, D, nb, dtype, dev)
    k, v, qd = kb.to(dev), vb.to(dev), q.to(dev)
    print(f"kv retrieval {dtype} D={D} R={R} T={T} K={K}", flush=True)
    kv_block_summary(k, S, L, 0, nb, kmin, kmax)
    sel = kv_select(qd, n, ret, kmin, kmax) if K else None
    o = kv_attention(qd, k, v, n, ret, sel)
    qr = q.float().transpose(1, 2)
    ref = ot.masked_attention(qr, kb.float(), vb.float(), ot.retrieval_mask(qr, kb.float(), ret))
    assert rel(o, ref) < tol(dtype)


class _Holder:
    """Stands in for the module the teacher is bound to (it reads ``self.retrieval``)."""

    def __init__(self, **ret):
        from heimdall_amd.teacher import set_retrieval
        self.retrieval = None
        if ret:
            set_retrieval(self, **ret)


def _teacher_inputs(seed, B, H, G, n, D, dtype):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, H, n, D, generator=g).to(dtype), torch.randn(B, G, n, D, generator=g).to(dtype),
            torch.randn(B, n, G, D, generator=g).to(dtype))


@pytest.mark.parametrize("dtype,D,ret", [
    (torch.bfloat16, 128, None),
    (torch.float32, 64, None),
    (torch.bfloat16, 128, dict(k=4, block=32, window=128, sinks=4)),
    (torch.bfloat16, 256, dict(k=8, block=16, window=64, sinks=2)),
    (torch.float32, 128, dict(k=0, block=32, window=100, sinks=4)),
])
def test_teacher_prefill_chunks_and_decode(dev, dtype, D, ret):
    """Prefill 600 tokens (t == n), a chunk of 40 (t < n, ring path), a chunk of 5 (split-K path), then 12 decode
    steps (retrieval when set), each against the oracle teacher with its own cache; the cache grows past its first
    capacity on the way."""
    from heimdall_amd.teacher import teacher
    B, H, G = 2, 8, 2
    qr, kr, v = _teacher_inputs(10, B, H, G, 657, D, dtype)
    m = _Holder(**(ret or {}))
    cache, ocache = {}, {}
    for lo, hi in [(0, 600), (600, 640), (640, 645)] + [(i, i + 1) for i in range(645, 657)]:
        print(f"teacher {dtype} D={D} ret={ret} tokens {lo}:{hi}", flush=True)
        o = teacher(m, qr[:, :, lo:hi].to(dev), kr[:, :, lo:hi].to(dev), v[:, lo:hi].to(dev), cache)
        ref = ot.teacher(qr[:, :, lo:hi].float(), kr[:, :, lo:hi].float(), v[:, lo:hi].float(), ocache, ret)
        assert o.dtype == dtype and o.shape == (B, hi - lo, H, D)
        assert rel(o, ref) < tol(dtype), (lo, hi, rel(o, ref))
        assert torch.equal(cache["k"].cpu().float(), ocache["k"].float())
        assert torch.equal(cache["v"].cpu().float(), ocache["v"].float())


def test_teacher_retrieval_prefill(dev):
    """prefill=True: every query of a 700-token prompt takes its own selection (queries inside the sinks see all
    sinks, as the reference's mask does)."""
    from heimdall_amd.teacher import teacher
    B, H, G, D, n = 1, 4, 2, 128, 700
    ret = dict(k=3, block=16, window=64, sinks=4, prefill=True)
    qr, kr, v = _teacher_inputs(11, B, H, G, n, D, torch.bfloat16)
    m = _Holder(**ret)
    o = teacher(m, qr.to(dev), kr.to(dev), v.to(dev), {})
    ref = ot.teacher(qr.float(), kr.float(), v.float(), {}, ret)
    assert rel(o, ref) < TOL16


def test_teacher_adopts_plain_cache(dev):
    """A cache whose "k" / "v" were written as plain tensors (the reference's torch.cat layout) is adopted; the
    retrieval summaries are rebuilt from it."""
    from heimdall_amd.teacher import teacher
    B, H, G, D, n = 1, 4, 1, 64, 400
    ret = dict(k=2, block=16, window=64, sinks=4)
    qr, kr, v = _teacher_inputs(12, B, H, G, n + 1, D, torch.float32)
    cache = {"k": kr[:, :, :n].to(dev), "v": v[:, :n].transpose(1, 2).to(dev)}
    m = _Holder(**ret)
    o = teacher(m, qr[:, :, n:].to(dev), kr[:, :, n:].to(dev), v[:, n:].to(dev), cache)
    ocache = {"k": kr[:, :, :n], "v": v[:, :n].transpose(1, 2)}
    ref = ot.teacher(qr[:, :, n:], kr[:, :, n:], v[:, n:], ocache, ret)
    assert rel(o, ref) < TOL32
    assert cache["k"].shape == (B, G, n + 1, D)
