"""The allocation-free decode entry point (bf_decode_fwd_noalloc) against bf_decode_fwd, through the C ABI.

Two calls in a row on fresh copies of the same cache, the second with a smaller batch and another geometry: outputs,
LSE, the updated state and the whole ring must be bit-identical to what bf_decode_fwd (same kernels, caller
workspace) writes. A problem larger than the static scratch is refused without a launch."""
import ctypes

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def make_step(B, H, G, D, W, S, pos, dtype, dev, seed):
    gen = torch.Generator(device=dev).manual_seed(seed)
    rn = lambda *s: torch.randn(*s, device=dev, generator=gen)
    ring_pos = torch.full((W,), -1, dtype=torch.long, device=dev)
    pp = torch.arange(max(0, pos - W), pos, device=dev)
    ring_pos[pp % W] = pp
    cache = dict(ring_k=rn(B, G, W, D).to(dtype), ring_v=rn(B, G, W, D).to(dtype),
                 ring_km=F.normalize(rn(B, W, G, D), dim=-1), ring_g=-torch.rand(B, W, G, device=dev, generator=gen),
                 ring_beta=torch.rand(B, W, G, device=dev, generator=gen), ring_pos=ring_pos,
                 state=rn(B, G, D, D) * 0.02)
    inp = dict(qr=rn(B, H, D).to(dtype), qm=F.normalize(rn(B, H, D), dim=-1) * D ** -0.5, kr=rn(B, G, D).to(dtype),
               v=rn(B, G, D).to(dtype), km=F.normalize(rn(B, G, D), dim=-1),
               g=-torch.rand(B, G, device=dev, generator=gen), beta=torch.rand(B, G, device=dev, generator=gen),
               z=rn(B, H), mix_lse=rn(H) * 0.3, mem_scale=torch.full((H,), D ** 0.5, device=dev),
               sink_k=rn(B, G, S, D).to(dtype), sink_v=rn(B, G, S, D).to(dtype))
    return cache, inp


def call(lib, fn, geom, cache, inp, ws=None):
    from heimdall_amd import _lib
    from heimdall_amd._device import dtype_code, stream_ptr
    B, H, G, D, W, S, pos = geom
    dt = dtype_code(inp["kr"].dtype)
    o = torch.empty(B, H, D, device=inp["qr"].device)
    lse = torch.empty(B, H, device=inp["qr"].device)
    p = lambda t: t.data_ptr()
    args = [B, G, H // G, D, W, S, pos, 1, dt, dt, p(inp["qr"]), p(inp["qm"]), p(inp["kr"]), p(inp["v"]), p(inp["km"]),
            p(inp["g"]), p(inp["beta"]), p(inp["z"]), p(inp["mix_lse"]), p(inp["mem_scale"]), p(inp["sink_k"]),
            p(inp["sink_v"]), S, p(cache["ring_k"]), p(cache["ring_v"]), p(cache["ring_km"]), p(cache["ring_g"]),
            p(cache["ring_beta"]), p(cache["ring_pos"]), p(cache["state"]), p(o), p(lse)]
    if fn == "bf_decode_fwd":
        args += [p(ws), ws.numel()]
    args.append(stream_ptr(inp["qr"].device))
    _lib.check(getattr(lib, fn)(*args), fn)
    return o, lse


@pytest.mark.parametrize("first,second", [((8, 16, 4, 256, 2048, 4, 5000), (3, 8, 2, 128, 512, 4, 700)),
                                          ((4, 24, 4, 256, 2048, 4, 2050), (1, 4, 1, 64, 64, 2, 65))])
def test_noalloc_decode_equals_workspace_decode(lib, dev, first, second):
    from heimdall_amd._device import workspace
    for i, geom in enumerate((first, second)):
        B, H, G, D, W, S, pos = geom
        print(f"noalloc decode call {i}: B={B} H={H} G={G} D={D} W={W} S={S} pos={pos}", flush=True)
        dtype = torch.bfloat16 if i == 0 else torch.float32
        cache_a, inp = make_step(B, H, G, D, W, S, pos, dtype, dev, seed=10 + i)
        cache_b = {k: v.clone() for k, v in cache_a.items()}
        n = ctypes.c_size_t(0)
        assert lib.bf_decode_workspace_size(B, G, H // G, D, W, ctypes.byref(n)) == 0
        o_a, lse_a = call(lib, "bf_decode_fwd", geom, cache_a, inp, workspace(n.value, dev))
        o_b, lse_b = call(lib, "bf_decode_fwd_noalloc", geom, cache_b, inp)
        torch.cuda.synchronize()
        assert torch.isfinite(o_a).all()
        assert torch.equal(o_a, o_b) and torch.equal(lse_a, lse_b)
        for k in cache_a:
            assert torch.equal(cache_a[k], cache_b[k]), k


def test_noalloc_decode_refuses_oversized_problem(lib):
    """B = 256 sequences of H = 32, D = 256, W = 8192 need more than the static scratch: BF_STATUS_SCRATCH, nothing
    launched (the check comes before any device call, so placeholder pointers are never touched)."""
    n = ctypes.c_size_t(0)
    assert lib.bf_decode_workspace_size(256, 4, 8, 256, 8192, ctypes.byref(n)) == 0 and n.value > 16 << 20
    fake = 256
    rc = lib.bf_decode_fwd_noalloc(256, 4, 8, 256, 8192, 4, 100000, 1, 1, 1, *([fake] * 12), 0, *([fake] * 9), None)
    assert rc == -4
    assert b"static scratch" in lib.bf_status_string(-4)
