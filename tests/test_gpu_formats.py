"""GPU parity of the llama.cpp state-row formats (``bf_llama_state_pack`` / ``bf_llama_state_unpack`` through
``heimdall_amd.formats``) against ``oracle.formats``: bit-exact rows (fp32 and bf16 rings, before and after the
window fills, sinks partly present), bit-exact round trips, and the production geometry."""
import numpy as np
import pytest
import torch

from oracle import formats as of

pytestmark = pytest.mark.gpu


def random_cache(B, G, D, W, S, n, seed, kv_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    c = dict(ring_k=torch.randn(B, G, W, D, generator=g).to(kv_dtype),
             ring_v=torch.randn(B, G, W, D, generator=g).to(kv_dtype),
             ring_km=torch.randn(B, W, G, D, generator=g), ring_g=-torch.rand(B, W, G, generator=g),
             ring_beta=torch.rand(B, W, G, generator=g), ring_pos=torch.full((W,), -1, dtype=torch.long),
             S=torch.randn(B, G, D, D, generator=g))
    for p in range(max(0, n - W), n):
        c["ring_pos"][p % W] = p
    ns = min(S, n)
    c["sink_k"] = torch.randn(B, G, ns, D, generator=g).to(kv_dtype)
    c["sink_v"] = torch.randn(B, G, ns, D, generator=g).to(kv_dtype)
    return c


def live(c):
    """The cache with the ring slots that hold no position zeroed (unpack writes zeros there)."""
    out = dict(c)
    dead = c["ring_pos"] < 0
    for key in ("ring_k", "ring_v"):
        out[key] = c[key].clone()
        out[key][:, :, dead] = 0
    for key in ("ring_km", "ring_g", "ring_beta"):
        out[key] = c[key].clone()
        out[key][:, dead] = 0
    return out


@pytest.mark.parametrize("kv_dtype,D,W,S,n", [(torch.float32, 64, 7, 2, 5), (torch.float32, 64, 7, 2, 30),
                                             (torch.bfloat16, 128, 40, 4, 3), (torch.bfloat16, 256, 33, 4, 500)])
def test_pack_matches_oracle_and_roundtrips(dev, kv_dtype, D, W, S, n):
    from heimdall_amd.formats import pack_llama_state, unpack_llama_state
    B, G = 2, 2
    c = random_cache(B, G, D, W, S, n, seed=n, kv_dtype=kv_dtype)
    print(f"llama state {kv_dtype} D={D} W={W} S={S} n={n}", flush=True)
    rows = pack_llama_state({k: v.to(dev) for k, v in c.items()}, n, W, S)
    want = np.stack([of.llama_state_row(c, b, n, W, S) for b in range(B)])
    assert np.array_equal(rows.cpu().numpy(), want)
    back = unpack_llama_state(rows, n, W, S, G, D, kv_dtype)
    want_c = live(c)
    for key in ("ring_k", "ring_v", "ring_km", "ring_g", "ring_beta", "ring_pos", "sink_k", "sink_v", "S"):
        assert torch.equal(back[key].cpu(), want_c[key]), key


def test_production_geometry_roundtrip(dev):
    """B = 8, G = 4, D = 256, W = 2048, S = 4 at position 100000 (43.7 MB rows): pack then unpack is exact."""
    from heimdall_amd.formats import llama_state_floats, pack_llama_state, unpack_llama_state
    B, G, D, W, S, n = 8, 4, 256, 2048, 4, 100000
    assert llama_state_floats(G, D, W, S) == 10_928_384
    c = {k: v.to(dev) for k, v in random_cache(B, G, D, W, S, n, seed=7, kv_dtype=torch.bfloat16).items()}
    rows = pack_llama_state(c, n, W, S)
    back = unpack_llama_state(rows, n, W, S, G, D, torch.bfloat16)
    for key in ("ring_k", "ring_v", "ring_km", "ring_g", "ring_beta", "ring_pos", "sink_k", "sink_v", "S"):
        assert torch.equal(back[key], c[key]), key
