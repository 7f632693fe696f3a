"""Decode for B sequences at different positions in one step (bf_decode_fwd_batch through hibrit.student_batch),
against the oracle run on each sequence alone: the llama.cpp multi-sequence setting (per-sequence positions in one
ubatch, Heimdall/llamacpp/bifrost.patch:841-884) and its own check (llamacpp/bifrost_multiseq.cpp:48-98): the batched
step equals one sequence at a time, a copied sequence continues like the original, and a reused row after its
sequence is removed behaves like a fresh sequence.

Positions cover the sinks (0, 1 with S = 2), the first window (9), the window edge (16 = W) and the ring after a
wrap (35); each sequence runs 12 steps from there. Tolerances (relative L2): <= 1e-4 fp32, <= 2e-2 bf16 cache."""
import pytest
import torch

from oracle import layer as olayer
from test_gpu_decode import make_core, make_inputs, rel, split, to_dev

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}
H, G, D, DM, W, S = 4, 2, 64, 32, 16, 2
STARTS = (0, 1, 9, 16, 35)
STEPS = 12


def _oracle_run(m, args, start, steps, cache=None):
    """The oracle on one sequence: a prefill of `start` tokens (one call) if the cache is new, then `steps` tokens one
    at a time; returns (outputs [1, steps, H, D], cache)."""
    c = {} if cache is None else cache
    argsf = tuple(z.float() for z in args)
    with torch.no_grad():
        if cache is None and start:
            olayer.student(m, *split(argsf, 0, start), 0, c)
        outs = [olayer.student(m, *split(argsf, t, t + 1), t, c) for t in range(start, start + steps)]
    return (torch.cat(outs, 1) if outs else None), c


def _join(a, b):
    """Two token ranges of one sequence (x, q, k, v along dim 1; qr, kr along dim 2) as one."""
    return tuple(torch.cat((u, w), dim) for u, w, dim in zip(a, b, (1, 1, 1, 1, 2, 2)))


def _stack(streams, at):
    """The token of each sequence at its own index at[i], stacked into a batch."""
    rows = [split(s, t, t + 1) for s, t in zip(streams, at)]
    return tuple(torch.cat([r[a] for r in rows], 0) for a in range(6))


def _check_row(mg, bc, i, pos, c_ref, tol):
    from heimdall_amd import hibrit
    cg = hibrit.batch_cache_get(mg, bc, i, pos)
    for key in ("ring_k", "ring_v", "ring_km", "ring_g", "ring_beta"):
        assert rel(cg[key], c_ref[key]) < tol, (i, key, rel(cg[key], c_ref[key]))
    assert torch.equal(cg["ring_pos"].cpu(), c_ref["ring_pos"]), i
    if c_ref.get("sink_k") is not None:
        assert rel(cg["sink_k"], c_ref["sink_k"]) < tol and rel(cg["sink_v"], c_ref["sink_v"]) < tol, i
    if c_ref.get("S") is not None:
        assert rel(cg["S"], c_ref["S"]) < tol, (i, rel(cg["S"], c_ref["S"]))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_batch_positions_equal_per_sequence(dev, dtype, margin):
    from heimdall_amd import hibrit
    print(f"batched decode, positions {STARTS} + {STEPS} steps, H={H} G={G} D={D} W={W} S={S} {dtype}", flush=True)
    m = make_core(H, G, D, DM, window=W, sinks=S)
    mg = make_core(H, G, D, DM, window=W, sinks=S).to(dev)
    streams = [make_inputs(m, 1, st + STEPS, seed=100 + i, dtype=dtype) for i, st in enumerate(STARTS)]
    refs = [_oracle_run(m, s, st, STEPS) for s, st in zip(streams, STARTS)]
    bc = hibrit.new_batch_cache(mg, len(STARTS), dtype, dev)
    with torch.no_grad():
        for i, (s, st) in enumerate(zip(streams, STARTS)):
            c = {}
            if st:
                hibrit.student(mg, *to_dev(split(s, 0, st), dev), 0, c)
            hibrit.batch_cache_set(mg, bc, i, c)
        outs = []
        for j in range(STEPS):
            pos = torch.tensor([st + j for st in STARTS], device=dev)
            outs.append(hibrit.student_batch(mg, *to_dev(_stack(streams, [st + j for st in STARTS]), dev), pos, bc))
    o = torch.cat(outs, 1).cpu()
    for i, st in enumerate(STARTS):
        margin(f"o, sequence at {st}..{st + STEPS - 1}, {dtype}", rel(o[i:i + 1], refs[i][0]), TOL[dtype])
        _check_row(mg, bc, i, st + STEPS, refs[i][1], TOL[dtype])


def test_batch_copied_and_reused_rows(dev):
    """Row 1 := a copy of row 0's cache, then both continue: row 1 (with its own tokens) equals the oracle continuing
    row 0's history with those tokens; row 2 is cleared (its sequence removed) and starts a fresh sequence at position
    0 beside the others: it equals a fresh oracle sequence."""
    from heimdall_amd import hibrit
    print("batched decode: copied row, reused row, fp32", flush=True)
    m = make_core(H, G, D, DM, window=W, sinks=S)
    mg = make_core(H, G, D, DM, window=W, sinks=S).to(dev)
    P = 30
    hist = make_inputs(m, 1, P, seed=7)
    cont = [make_inputs(m, 1, STEPS, seed=8 + i) for i in range(3)]
    # oracle: row 0's history, continued with cont[0]; the same history continued with cont[1]; a fresh sequence
    _, c0 = _oracle_run(m, hist, P, 0)
    import copy
    c1 = copy.deepcopy(c0)
    full0, full1 = _join(hist, cont[0]), _join(hist, cont[1])
    ref0, _ = _oracle_run(m, full0, P, STEPS, c0)
    ref1, _ = _oracle_run(m, full1, P, STEPS, c1)
    ref2, _ = _oracle_run(m, cont[2], 0, STEPS)
    bc = hibrit.new_batch_cache(mg, 3, torch.float32, dev)
    with torch.no_grad():
        c = {}
        hibrit.student(mg, *to_dev(hist, dev), 0, c)
        hibrit.batch_cache_set(mg, bc, 0, c)
        hibrit.batch_cache_set(mg, bc, 2, c)                                     # an old sequence, then removed:
        hibrit.batch_cache_set(mg, bc, 1, hibrit.batch_cache_get(mg, bc, 0, P))  # row 1 := row 0
        hibrit.batch_cache_set(mg, bc, 2, None)                                  # row 2 cleared, reused below
        outs = []
        for j in range(STEPS):
            pos = torch.tensor([P + j, P + j, j], device=dev)
            outs.append(hibrit.student_batch(mg, *to_dev(_stack(cont, [j, j, j]), dev), pos, bc))
    o = torch.cat(outs, 1).cpu()
    for i, ref in enumerate((ref0, ref1, ref2)):
        e = rel(o[i:i + 1], ref)
        print(f"  row {i} rel err {e:.2e}", flush=True)
        assert e < 1e-4, (i, e)


def test_batch_shared_position_matches_decode(dev):
    """B = 3 sequences that share one position through bf_decode_fwd_batch give the bits of bf_decode_fwd on the same
    cache (the shared-position entry), past the window with the memory active."""
    from heimdall_amd import hibrit
    print("batched decode at one shared position vs bf_decode_fwd, bf16", flush=True)
    m = make_core(H, G, D, DM, window=W, sinks=S)
    mg = make_core(H, G, D, DM, window=W, sinks=S).to(dev)
    P, B = 40, 3
    args = to_dev(make_inputs(m, B, P + 3, seed=21, dtype=torch.bfloat16), dev)
    with torch.no_grad():
        c = {}
        hibrit.student(mg, *split(args, 0, P), 0, c)
        bc = hibrit.new_batch_cache(mg, B, torch.bfloat16, dev)
        for i in range(B):
            hibrit.batch_cache_set(mg, bc, i, {key: (val[i:i + 1] if torch.is_tensor(val) and val.dim() > 1 and
                                                     key != "ring_pos" else val) for key, val in c.items()})
        for t in range(P, P + 3):
            o_ref = hibrit.student(mg, *split(args, t, t + 1), t, c)
            o = hibrit.student_batch(mg, *split(args, t, t + 1), torch.full((B,), t, device=dev), bc)
            assert torch.equal(o, o_ref), (t, rel(o, o_ref))
