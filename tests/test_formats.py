"""Host-side conversion formats of ``heimdall_amd.formats`` (parameter reshuffles, no kernels): the GGUF tensors of a
converted core against the oracle's (``oracle.formats.gguf_tensors``, restating ``bifrost_gguf.py:24-47``), their
round trip into a fresh core, and the conversion dict of ``HybridLM.conversion_state`` / ``apply_conversion``."""
import torch

from heimdall_amd import formats
from heimdall_amd.hibrit import BifrostCore, CoreConfig
from oracle import formats as of


def converted_core(seed=0, archival=1):
    torch.manual_seed(seed)
    core = BifrostCore(CoreConfig(h=8, hkv=4, dh=16, d=32))
    core.convert(window=64, sinks=4, archival=archival)
    with torch.no_grad():
        for p in core.parameters():
            p.add_(torch.randn_like(p) * 0.1)
    return core


def test_gguf_tensors_match_oracle():
    core = converted_core()
    got = formats.gguf_tensors(core, layer=3)
    params = {n: p for n, p in core.named_parameters()}
    want = of.gguf_tensors(params, archival=1)
    assert set(got) == {f"blk.3.{k}" for k in want}
    for k, v in want.items():
        assert torch.equal(got[f"blk.3.{k}"], v), k


def test_gguf_roundtrip_into_fresh_core():
    core = converted_core(seed=1, archival=2)
    t = formats.gguf_tensors(core, layer=0)
    fresh = BifrostCore(CoreConfig(h=8, hkv=4, dh=16, d=32))
    formats.load_gguf_tensors(fresh, t, layer=0, window=64, sinks=4)
    assert int((fresh.decay_mask == 0).sum()) == 2
    for name, p in core.named_parameters():
        q = dict(fresh.named_parameters())[name]
        if name == "A_log":                    # not stored for the archival heads (masked out)
            assert torch.allclose(q[2:], p[2:], rtol=1e-6)
        else:
            assert torch.equal(q, p), name
    # the round trip reproduces the tensors exactly
    t2 = formats.gguf_tensors(fresh, layer=0)
    for k in t:
        assert torch.allclose(t2[k], t[k], rtol=1e-6, atol=0), k


def test_conversion_dict_roundtrip():
    cores = {"layers.3": converted_core(seed=2), "layers.7": converted_core(seed=3, archival=0)}
    st = formats.conversion_state(cores, meta={"note": "x"})
    assert [c["name"] for c in st["conv"]] == ["layers.3", "layers.7"]
    assert st["conv"][0] == dict(name="layers.3", window=64, sinks=4, archival=1)
    assert "layers.3.self_attn.ab.weight" in st["params"] and "layers.7.self_attn.A_log" in st["params"]
    fresh = {n: BifrostCore(CoreConfig(h=8, hkv=4, dh=16, d=32)) for n in cores}
    formats.apply_conversion(fresh, st)
    for n in cores:
        for name, p in cores[n].named_parameters():
            assert torch.equal(dict(fresh[n].named_parameters())[name], p), (n, name)
        assert torch.equal(fresh[n].decay_mask, cores[n].decay_mask)
