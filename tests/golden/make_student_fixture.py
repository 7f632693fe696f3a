"""Writes ``student_tiny.npz``: inputs, parameters and outputs of the reference's own
``HybridAttention._student`` (``Heimdall/heimdall/hibrit.py:363-424``) on a tiny converted layer with trained-like
parameters, run once over chunk splits with a cache (5,1,13,1,1,9,30,1 — the split of
``Heimdall/tests/test_hibrit.py:86``) and once without a cache.

Run in the build container only (the reference is not shipped anywhere):

    python tests/golden/make_student_fixture.py /root/reference

The fixture is data (inputs and expected outputs); no reference source is copied.
"""
import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "student_tiny.npz"


def main(ref_root: str) -> None:
    sys.path.insert(0, str(Path(ref_root) / "Heimdall"))
    from heimdall.hibrit import HybridAttention, HybridConfig

    text = dict(model_type="qwen3_5_text", vocab_size=32, hidden_size=16, intermediate_size=32, num_hidden_layers=4,
                num_attention_heads=4, num_key_value_heads=2, head_dim=8, linear_num_key_heads=2,
                linear_num_value_heads=2, linear_key_head_dim=8, linear_value_head_dim=8, linear_conv_kernel_dim=4,
                full_attention_interval=4, attn_output_gate=True, rms_norm_eps=1e-6, hidden_act="silu",
                rope_parameters={"rope_type": "default", "rope_theta": 10000.0, "partial_rotary_factor": 0.25})
    cfg = HybridConfig(text)
    torch.manual_seed(0)
    a = HybridAttention(cfg)
    a.convert(window=8, sinks=2, archival=1)
    gen = torch.Generator().manual_seed(1)
    with torch.no_grad():
        for lin in (a.ab, a.mix):
            lin.weight.add_(torch.randn(lin.weight.shape, generator=gen) * 0.3)
            lin.bias.add_(torch.randn(lin.bias.shape, generator=gen) * 0.3)
        a.mix.bias.fill_(0.5)
        a.fq.add_(torch.randn(a.fq.shape, generator=gen) * 0.1)
        a.fk.add_(torch.randn(a.fk.shape, generator=gen) * 0.1)
        a.mix_lse.copy_(torch.randn(a.mix_lse.shape, generator=gen) * 0.3)
    b, t, H, G, D, d = 2, 61, 4, 2, 8, 16
    x = torch.randn(b, t, d, generator=gen)
    q = torch.randn(b, t, H, D, generator=gen)
    k = torch.randn(b, t, G, D, generator=gen)
    v = torch.randn(b, t, G, D, generator=gen)
    qr = torch.randn(b, H, t, D, generator=gen)
    kr = torch.randn(b, G, t, D, generator=gen)
    splits = (5, 1, 13, 1, 1, 9, 30, 1)
    with torch.no_grad():
        cache, outs, s = {}, [], 0
        for n in splits:
            outs.append(a._student(x[:, s:s + n], q[:, s:s + n], k[:, s:s + n], v[:, s:s + n],
                                   qr[:, :, s:s + n], kr[:, :, s:s + n], s, cache))
            s += n
        o = torch.cat(outs, 1)
        o_full = a._student(x, q, k, v, qr, kr, 0, None)
    f = lambda z: z.detach().float().numpy()
    np.savez_compressed(
        OUT, h=H, hkv=G, dh=D, d=d, window=a.window, sinks=a.sinks, splits=np.array(splits),
        fq=f(a.fq), fk=f(a.fk), ab_w=f(a.ab.weight), ab_b=f(a.ab.bias), mix_w=f(a.mix.weight), mix_b=f(a.mix.bias),
        mix_lse=f(a.mix_lse), mem_scale=f(a.mem_scale), A_log=f(a.A_log), dt_bias=f(a.dt_bias),
        decay_mask=f(a.decay_mask), x=f(x), q=f(q), k=f(k), v=f(v), qr=f(qr), kr=f(kr), o=f(o), o_full=f(o_full),
        S=f(cache["S"]), ring_pos=cache["ring_pos"].numpy())
    print("wrote", OUT, OUT.stat().st_size, "bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
