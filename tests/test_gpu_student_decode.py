"""The fused decode entry bf_student_decode (gate and memory projections, gates and the decode step in one call)
against the same step composed from bf_gate_project, bf_mem_project, bf_mem_gates and bf_decode_fwd /
bf_decode_fwd_batch: the same kernels on the same values, so outputs and caches must match bit for bit (for dense
step inputs: a strided x sends the composed path's gate projection to PyTorch's fp32 GEMM instead). Steps start
at position 0 (sinks filling, S = 2), cross the window edge (W = 16: the memory switches on) and run past the ring
wrap; the batched form covers sequences at different positions. The oracle parity of the decode step itself is
covered by test_gpu_decode.py and test_gpu_decode_batch.py, which now run through this entry."""
import pytest
import torch

from test_gpu_decode import make_core, make_inputs, split, to_dev

pytestmark = pytest.mark.gpu

H, G, D, DM, W, S = 4, 2, 64, 32, 16, 2
STEPS = 40


def _run(dev, fused: bool, monkeypatch):
    from heimdall_amd import hibrit
    if not fused:
        monkeypatch.setattr(hibrit, "_fused_decode_ok", lambda *a, **k: False)
    mg = make_core(H, G, D, DM, window=W, sinks=S).to(dev)
    args = to_dev(make_inputs(mg, 2, STEPS, seed=5, dtype=torch.bfloat16), dev)
    c, outs = {}, []
    with torch.no_grad():
        for t in range(STEPS):
            step = tuple(z_.contiguous() for z_ in split(args, t, t + 1))   # dense, as a decode loop feeds
            outs.append(hibrit.student(mg, *step, t, c))
    monkeypatch.undo()
    return torch.cat(outs, 1), c


def test_fused_decode_equals_composed(dev, monkeypatch):
    print(f"student decode, fused vs composed, {STEPS} steps from position 0, H={H} G={G} D={D} W={W} S={S}",
          flush=True)
    o1, c1 = _run(dev, True, monkeypatch)
    o0, c0 = _run(dev, False, monkeypatch)
    assert torch.equal(o1, o0)
    for key in ("sink_k", "sink_v", "ring_k", "ring_v", "ring_km", "ring_g", "ring_beta", "ring_pos", "S"):
        assert torch.equal(c1[key], c0[key]), key


def test_fused_batch_decode_equals_composed(dev, monkeypatch):
    from heimdall_amd import hibrit
    print("student_batch, fused vs composed, sequences at positions 0, 3, 15, 30", flush=True)
    starts = (0, 3, 15, 30)
    res = []
    for fused in (True, False):
        if not fused:
            monkeypatch.setattr(hibrit, "_fused_decode_ok", lambda *a, **k: False)
        mg = make_core(H, G, D, DM, window=W, sinks=S).to(dev)
        streams = [to_dev(make_inputs(make_core(H, G, D, DM, window=W, sinks=S), 1, st + 6, seed=40 + i,
                                      dtype=torch.bfloat16), dev) for i, st in enumerate(starts)]
        bc = hibrit.new_batch_cache(mg, len(starts), torch.bfloat16, dev)
        outs = []
        with torch.no_grad():
            for i, (sq, st) in enumerate(zip(streams, starts)):
                c = {}
                if st:
                    hibrit.student(mg, *split(sq, 0, st), 0, c)
                hibrit.batch_cache_set(mg, bc, i, c)
            for j in range(6):
                rows = [split(sq, st + j, st + j + 1) for sq, st in zip(streams, starts)]
                batch = tuple(torch.cat([r_[a] for r_ in rows], 0) for a in range(6))
                pos = torch.tensor([st + j for st in starts], device=dev)
                outs.append(hibrit.student_batch(mg, *batch, pos, bc))
        monkeypatch.undo()
        res.append((torch.cat(outs, 1), bc))
    (o1, b1), (o0, b0) = res
    assert torch.equal(o1, o0)
    for key in hibrit.BATCH_KEYS:
        assert torch.equal(b1[key], b0[key]), key


def test_fused_decode_rejects_bad_arguments(dev):
    """The entry validates its sizes and pointers before launching anything."""
    from heimdall_amd import _lib
    lib = _lib.load()
    n = _lib.ctypes.c_size_t(0)
    assert lib.bf_student_decode_workspace_size(1, 6, 4, 64, 16, 32, _lib.ctypes.byref(n)) != 0  # H % G != 0
    assert lib.bf_student_decode_workspace_size(1, 8, 4, 64, 16, 32, _lib.ctypes.byref(n)) == 0
    assert n.value > 0
    args = [1, 8, 4, 64, 16, 2, 5, None, 1, 30] + [None] * 19 + [0] + [None] * 9 + [n.value, None]
    assert lib.bf_student_decode(*args) != 0                       # d_model not a multiple of 8, null pointers
