"""Oracle: the formats around the converted layer (test infrastructure only — see ``oracle/__init__.py``).

- The llama.cpp per-sequence state row of a converted layer (``Heimdall/llamacpp/bifrost.patch``: the sizes
  ``bifrost_ring_ch`` / ``bifrost_region`` / ``bifrost_state`` at :221-239, the slot rule "slot = S + pos mod (W+1)"
  at :816-827, the views region / K plane / V plane / delta of ``build_layer_bifrost`` at :1000-1013), built slot by
  slot from the student cache of ``HybridAttention._student`` (``Heimdall/heimdall/hibrit.py:363-424``), and back.
- The GGUF tensors of a conversion (``Heimdall/llamacpp/bifrost_gguf.py:24-47``, ``tensors_from_conv``): per layer
  ``blk.N.bifrost_{fq,fk,ab,ab_b,mix,mix_b,mix_lse,mem_scale,a,dt}``, and back.

Pins (``tests/test_oracle_formats.py``): the row size at the production geometry against the value the patch's
formula gives (10,928,384 floats at G=4, D=256, W=2048, S=4); the delta block read with ggml's mul_mat convention
reproduces o = q S; the GGUF tensors used the way llama.cpp's graph uses them reproduce the reference's memory
inputs (g = A softplus(a + dt) with A = -e^A_log masked, qm from the transposed fq); round trips.
"""
import numpy as np
import torch


def region_slots(W: int, S: int) -> int:
    """LR: sinks + ring of W + 1 + scratch, rounded up to 32 (``bifrost.patch:229-231``)."""
    return (S + W + 2 + 31) // 32 * 32


def ring_channels(G: int, D: int) -> int:
    """C = 3 G D + 2 G: [k_rope | v | k_mem | g | beta] (``bifrost.patch:224-227``)."""
    return 3 * G * D + 2 * G


def state_floats(G: int, D: int, W: int, S: int) -> int:
    """``bifrost_state``: region * (C + 2 G D) + D^2 G (``bifrost.patch:233-239``)."""
    return region_slots(W, S) * (ring_channels(G, D) + 2 * G * D) + D * D * G


def llama_state_row(cache: dict, b: int, n: int, W: int, S: int) -> np.ndarray:
    """The row of sequence b after n tokens, float32, from a student cache (numpy arrays or CPU tensors)."""
    c = {k: (v.float().numpy() if torch.is_tensor(v) and v.is_floating_point() else
             (v.numpy() if torch.is_tensor(v) else v)) for k, v in cache.items()}
    G, D = c["ring_k"].shape[1], c["ring_k"].shape[3]
    LR, C, GD = region_slots(W, S), ring_channels(G, D), G * D
    region = np.zeros((LR, C), np.float32)
    lo = max(0, n - W)
    ns = 0 if c.get("sink_k") is None else c["sink_k"].shape[2]

    def ring_row(p):
        s = p % W
        if p < lo or p >= n or int(c["ring_pos"][s]) != p:
            return None
        return (c["ring_k"][b, :, s].reshape(GD), c["ring_v"][b, :, s].reshape(GD), c["ring_km"][b, s].reshape(GD),
                c["ring_g"][b, s], c["ring_beta"][b, s])

    for j in range(min(S, ns)):                               # sinks: slots 0 .. S - 1
        region[j, :GD] = c["sink_k"][b, :, j].reshape(GD)
        region[j, GD:2 * GD] = c["sink_v"][b, :, j].reshape(GD)
        r = ring_row(j)
        if r is not None:
            region[j, 2 * GD:] = np.concatenate((r[2], r[3], r[4]))
    for p in range(lo, n):                                    # the window: slot S + p mod (W + 1)
        r = ring_row(p)
        if r is not None:
            region[S + p % (W + 1)] = np.concatenate(r)
    kplane = region[:, :GD].reshape(LR, G, D).transpose(1, 0, 2)           # [G][LR][D]
    vplane = region[:, GD:2 * GD].reshape(LR, G, D).transpose(1, 2, 0)     # [G][D][LR]
    delta = c["S"][b].transpose(0, 2, 1)                                   # [G][dv][dk]
    return np.concatenate((region.ravel(), kplane.ravel(), vplane.ravel(), delta.ravel())).astype(np.float32)


def cache_from_llama_rows(rows: np.ndarray, n: int, W: int, S: int, G: int, D: int) -> dict:
    """The student cache (float32 numpy) from rows [B][floats]: the ring holds positions max(0, n - W) .. n - 1 at
    slot p mod W, the sinks the first min(S, n) slots."""
    B = rows.shape[0]
    LR, C, GD = region_slots(W, S), ring_channels(G, D), G * D
    out = dict(ring_k=np.zeros((B, G, W, D), np.float32), ring_v=np.zeros((B, G, W, D), np.float32),
               ring_km=np.zeros((B, W, G, D), np.float32), ring_g=np.zeros((B, W, G), np.float32),
               ring_beta=np.zeros((B, W, G), np.float32), ring_pos=np.full(W, -1, np.int64))
    ns = min(S, n)
    out["sink_k"] = np.zeros((B, G, ns, D), np.float32)
    out["sink_v"] = np.zeros((B, G, ns, D), np.float32)
    out["S"] = np.zeros((B, G, D, D), np.float32)
    for b in range(B):
        region = rows[b, :LR * C].reshape(LR, C)
        for p in range(max(0, n - W), n):
            s, row = p % W, region[S + p % (W + 1)]
            out["ring_k"][b, :, s] = row[:GD].reshape(G, D)
            out["ring_v"][b, :, s] = row[GD:2 * GD].reshape(G, D)
            out["ring_km"][b, s] = row[2 * GD:3 * GD].reshape(G, D)
            out["ring_g"][b, s] = row[3 * GD:3 * GD + G]
            out["ring_beta"][b, s] = row[3 * GD + G:]
            out["ring_pos"][s] = p
        for j in range(ns):
            out["sink_k"][b, :, j] = region[j, :GD].reshape(G, D)
            out["sink_v"][b, :, j] = region[j, GD:2 * GD].reshape(G, D)
        off = LR * C + 2 * LR * GD
        out["S"][b] = rows[b, off:off + G * D * D].reshape(G, D, D).transpose(0, 2, 1)
    return out


def gguf_tensors(params: dict, archival: int) -> dict:
    """The GGUF tensors of one converted layer from its parameters (the conversion dict's ``<layer>.self_attn.*``
    entries without the prefix): fq / fk transposed per head (ggml's mul_mat contracts a tensor's first axis), the
    a = -e^A_log with the archival heads zeroed (never decaying), the rest as stored (``bifrost_gguf.py:31-41``)."""
    f = lambda k: params[k].detach().float().cpu()
    mask = torch.ones_like(f("A_log"))
    mask[:archival] = 0.0
    return {"bifrost_fq": f("fq").transpose(1, 2).contiguous(), "bifrost_fk": f("fk").transpose(1, 2).contiguous(),
            "bifrost_ab": f("ab.weight"), "bifrost_ab_b": f("ab.bias"), "bifrost_mix": f("mix.weight"),
            "bifrost_mix_b": f("mix.bias"), "bifrost_mix_lse": f("mix_lse"), "bifrost_mem_scale": f("mem_scale"),
            "bifrost_a": -f("A_log").exp() * mask, "bifrost_dt": f("dt_bias")}
