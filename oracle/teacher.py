"""Oracle: attention of the kept full-attention layers over a KV cache, with Quest-style retrieval (test
infrastructure only — see ``oracle/__init__.py``).

Restates ``HybridAttention._teacher`` (``Heimdall/heimdall/hibrit.py:275-290``) and ``_retrieval_mask``
(``hibrit.py:301-324``) on the host: the block summaries, the per-query candidate count, the top-k selection per KV
head, the attended-key mask and the masked softmax attention, in fp64.

Pins (``tests/test_oracle_teacher.py``): the mask against a per-query brute-force selection written from the
definition in ``set_retrieval``'s docstring (``hibrit.py:293-299``; the reference's own check is
``Heimdall/tests/test_hibrit.py:245-270``); k covering every block gives the causal mask (the reference's
``test_retrieval_all_blocks_equals_full``, ``test_hibrit.py:231-242``); k = 0 keeps only the sinks and the window;
``teacher`` without retrieval against ``torch.nn.functional.scaled_dot_product_attention`` (causal and prefix masks),
and decode with a growing cache against one call over the whole sequence.
"""
from typing import Optional

import torch


def block_summary(kr: torch.Tensor, sinks: int, block: int):
    """kr [B, G, n, D] -> per-dimension key minimum and maximum of the nb = (n - S) / L full blocks after the sinks,
    [B, G, nb, D] each (fp64)."""
    B, G, n, D = kr.shape
    nb = max(0, (n - sinks) // block)
    kb = kr[:, :, sinks:sinks + nb * block].double().reshape(B, G, nb, block, D)
    return kb.min(3).values, kb.max(3).values


def upper_bounds(qr: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor) -> torch.Tensor:
    """qr [B, H, t, D], kmin / kmax [B, G, nb, D] -> [B, G, t, nb]: for each KV head, the maximum over its R query
    heads of sum_d max(q_d kmin_d, q_d kmax_d), an upper bound on q.k for every key of the block."""
    B, H, t, D = qr.shape
    G = kmin.shape[1]
    q = qr.double().reshape(B, G, H // G, t, 1, D)
    lo, hi = kmin[:, :, None, None], kmax[:, :, None, None]            # [B, G, 1, 1, nb, D]
    ub = torch.maximum(q * lo, q * hi).sum(-1)                          # [B, G, R, t, nb]
    return ub.max(2).values


def candidates(n: int, t: int, sinks: int, window: int, block: int) -> torch.Tensor:
    """Candidate blocks of the queries at positions n - t .. n - 1: the blocks that end before the window,
    nc = min(max(p - W + 1 - S, 0) // L, nb). Returns nc [t] (int64)."""
    nb = max(0, (n - sinks) // block)
    p = torch.arange(n - t, n)
    return torch.clamp(torch.clamp(p - window + 1 - sinks, min=0) // block, max=nb)


def select_blocks(qr: torch.Tensor, kr: torch.Tensor, k: int, block: int, window: int, sinks: int):
    """The selected blocks: for each (b, g, query), the k candidates with the highest upper bound (ties to the lower
    block id). Returns (sel bool [B, G, t, nb], nc [t])."""
    B, H, t, D = qr.shape
    n = kr.shape[2]
    kmin, kmax = block_summary(kr, sinks, block)
    nb = kmin.shape[2]
    nc = candidates(n, t, sinks, window, block)
    sel = torch.zeros(B, kr.shape[1], t, nb, dtype=torch.bool)
    if nb == 0 or k == 0:
        return sel, nc
    ub = upper_bounds(qr, kmin, kmax)
    for i in range(t):
        c = int(nc[i])
        if c == 0:
            continue
        u = ub[:, :, i, :c]
        # stable descending order: equal bounds keep the lower block id first
        order = torch.sort(-u, dim=-1, stable=True).indices[..., :k]
        sel[:, :, i].scatter_(-1, order, True)
    return sel, nc


def retrieval_mask(qr: torch.Tensor, kr: torch.Tensor, ret: dict) -> torch.Tensor:
    """Boolean mask [B, H, t, n] (True = attend) of the last t queries over the n cached keys: the sinks (every key
    before S, also past a query that sits inside them), the selected blocks, and the window from the block
    boundary S + nc L to the query's own position."""
    B, H, t, D = qr.shape
    G, n = kr.shape[1], kr.shape[2]
    S, W, L, K = ret["sinks"], ret["window"], ret["block"], ret["k"]
    sel, nc = select_blocks(qr, kr, K, L, W, S)
    nb = sel.shape[-1]
    mask = torch.zeros(B, G, t, n, dtype=torch.bool)
    mask[..., :S] = True
    for i in range(t):
        p = n - t + i
        mask[:, :, i, S + int(nc[i]) * L:p + 1] = True
        for j in range(nb):
            m = sel[:, :, i, j]
            if m.any():
                mask[:, :, i, S + j * L:S + (j + 1) * L] |= m[..., None]
    return mask.repeat_interleave(H // G, dim=1)


def uses_retrieval(ret: Optional[dict], t: int, n: int) -> bool:
    """The teacher takes the retrieval mask for single-token decode (or any t with prefill on) once the context holds
    the sinks, the window and k full blocks (``hibrit.py:281``)."""
    return ret is not None and (t == 1 or bool(ret.get("prefill"))) and \
        n - ret["sinks"] - ret["window"] >= ret["k"] * ret["block"]


def teacher_mask(qr: torch.Tensor, kr: torch.Tensor, ret: Optional[dict]) -> torch.Tensor:
    """The mask the teacher applies [B, H, t, n]: retrieval when ``uses_retrieval``, else each query sees the keys up
    to its own position (causal for t == n)."""
    B, H, t, _ = qr.shape
    n = kr.shape[2]
    if uses_retrieval(ret, t, n):
        return retrieval_mask(qr, kr, ret)
    p = torch.arange(n - t, n)
    m = torch.arange(n)[None, :] <= p[:, None]
    return m[None, None].expand(B, H, t, n)


def masked_attention(qr: torch.Tensor, kr: torch.Tensor, vt: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """softmax(q k^T / sqrt(D) + log mask) v with grouped KV heads, fp64. qr [B, H, t, D], kr / vt [B, G, n, D],
    mask [B, H, t, n] -> o [B, t, H, D]."""
    B, H, t, D = qr.shape
    G = kr.shape[1]
    k = kr.double().repeat_interleave(H // G, dim=1)
    v = vt.double().repeat_interleave(H // G, dim=1)
    s = qr.double() @ k.transpose(-1, -2) * D ** -0.5
    s = s.masked_fill(~mask, float("-inf"))
    return (torch.softmax(s, dim=-1) @ v).transpose(1, 2)


def teacher(qr: torch.Tensor, kr: torch.Tensor, v: torch.Tensor, cache: Optional[dict],
            ret: Optional[dict] = None) -> torch.Tensor:
    """``_teacher(qr, kr, v, cache)``: qr [B, H, t, D], kr [B, G, t, D], v [B, t, G, D]; the cache's "k" / "v"
    [B, G, n, D] grow by the new rows. Returns o [B, t, H, D] (fp64)."""
    vt = v.transpose(1, 2)
    if cache is not None:
        if "k" in cache:
            kr, vt = torch.cat((cache["k"], kr), 2), torch.cat((cache["v"], vt), 2)
        cache["k"], cache["v"] = kr, vt
    return masked_attention(qr, kr, vt, teacher_mask(qr, kr, ret))
