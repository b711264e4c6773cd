"""CPU restatement of document-masked GQA attention (test oracle, float64).

Reference: ``packbalance/model/attention.py``
  * mask of the FlexAttention path:  doc[q] == doc[kv] and q >= kv   (:43-44)
    -- padding tokens (doc_id = -1) form one more "document";
  * ``eager_attention`` (:66-95): per document id >= 0, causal SDPA on that
    document's tokens; rows with doc_id < 0 stay 0;
  * GQA: query head h reads KV head h // (Hq/Hkv)  (repeat_interleave, :75-78;
    ``enable_gqa`` in flex, :121); softmax scale 1/sqrt(D).

``attention`` computes the forward (out, lse) and, given dO, the gradients
with the standard closed forms
    P = softmax(S), dV = P^T dO, dP = dO V^T, dS = P*(dP - rowsum(dO*O)),
    dQ = scale*dS K, dK = scale*dS^T Q
processed in query-row chunks so cfg-sized packs fit in host memory.  The
closed forms are pinned against torch autograd in tests/test_oracle.py.
"""

from __future__ import annotations

import math

import torch


def _chunk_rows(heads: int, keys: int, budget_bytes: int = 1 << 27) -> int:
    per_row = max(1, heads * keys * 8)
    return max(16, min(4096, budget_bytes // per_row))


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, doc_ids: torch.Tensor,
              dout: torch.Tensor | None = None, *, semantics: str = "flex",
              scale: float | None = None, dtype: torch.dtype = torch.float64,
              delta_out: torch.Tensor | None = None):
    """Document-masked causal GQA attention in float64.

    q [B, Hq, S, D], k/v [B, Hkv, S, D], doc_ids [B, S] (int), dout like q.
    semantics: "flex"  -> mask_mod of attention.py:43-44 (pads attend to pads);
               "eager" -> eager_attention of attention.py:66-95 (pad rows are 0
                          and never attend or get attended).
    delta_out: the output whose rowsum(dO * O) enters dS (default: the exact
               O computed here).  A backward reads its forward's STORED output,
               so passing a bf16 output models what any bf16-output
               implementation computes (FlexAttention's backward included:
               its delta is rowsum(dO * OUT) of the stored OUT).
    Returns dict with out [B,Hq,S,D], lse [B,Hq,S] (natural log; -inf on rows
    with no allowed key) and, if dout is given, dq, dk, dv (CPU, ``dtype``;
    float64 unless a caller trades precision for speed on large packs).
    """
    if semantics not in ("flex", "eager"):
        raise ValueError(semantics)
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if Hq % Hkv:
        raise ValueError("Hq must be a multiple of Hkv")
    G = Hq // Hkv
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    dev = "cpu"
    Q = q.detach().to(dev, dtype)
    K = k.detach().to(dev, dtype).repeat_interleave(G, dim=1)
    V = v.detach().to(dev, dtype).repeat_interleave(G, dim=1)
    dO = None if dout is None else dout.detach().to(dev, dtype)
    Od = None if delta_out is None else delta_out.detach().to(dev, dtype)
    docs = doc_ids.detach().to(dev, torch.int64).reshape(B, S)

    out = torch.zeros(B, Hq, S, D, dtype=dtype)
    lse = torch.full((B, Hq, S), -math.inf, dtype=dtype)
    dq = torch.zeros_like(out) if dO is not None else None
    dk_full = torch.zeros(B, Hq, S, D, dtype=dtype) if dO is not None else None
    dv_full = torch.zeros_like(dk_full) if dO is not None else None

    pos = torch.arange(S)
    for b in range(B):
        doc = docs[b]
        # For each query row, the first key it may see: the earliest key
        # position with the same document id (general doc layouts allowed).
        first = torch.empty(S, dtype=torch.int64)
        seen: dict[int, int] = {}
        for i, d in enumerate(doc.tolist()):
            first[i] = seen.setdefault(d, i)
        step = _chunk_rows(Hq, S)
        for r0 in range(0, S, step):
            r1 = min(S, r0 + step)
            lo = int(first[r0:r1].min())
            qi = pos[r0:r1]
            ki = pos[lo:r1]
            allowed = (doc[r0:r1, None] == doc[None, lo:r1]) & (qi[:, None] >= ki[None, :])
            if semantics == "eager":
                allowed &= (doc[r0:r1, None] >= 0) & (doc[None, lo:r1] >= 0)
            s = torch.einsum("hqd,hkd->hqk", Q[b, :, r0:r1], K[b, :, lo:r1]) * sc
            s = s.masked_fill(~allowed[None], -math.inf)
            m = s.amax(dim=-1, keepdim=True)
            has = torch.isfinite(m)
            m = torch.where(has, m, torch.zeros_like(m))
            p = torch.exp(s - m)
            l = p.sum(dim=-1, keepdim=True)
            p = torch.where(has, p / torch.where(has, l, torch.ones_like(l)), torch.zeros_like(p))
            o = torch.einsum("hqk,hkd->hqd", p, V[b, :, lo:r1])
            out[b, :, r0:r1] = o
            lse[b, :, r0:r1] = torch.where(has[..., 0], (m + torch.log(l))[..., 0],
                                           torch.full_like(m[..., 0], -math.inf))
            if dO is not None:
                do = dO[b, :, r0:r1]
                dp = torch.einsum("hqd,hkd->hqk", do, V[b, :, lo:r1])
                od = o if Od is None else Od[b, :, r0:r1]
                delta = (do * od).sum(dim=-1, keepdim=True)
                ds = p * (dp - delta)
                dq[b, :, r0:r1] = torch.einsum("hqk,hkd->hqd", ds, K[b, :, lo:r1]) * sc
                dk_full[b, :, lo:r1] += torch.einsum("hqk,hqd->hkd", ds, Q[b, :, r0:r1]) * sc
                dv_full[b, :, lo:r1] += torch.einsum("hqk,hqd->hkd", p, do)
    res = {"out": out, "lse": lse}
    if dO is not None:
        res["dq"] = dq
        res["dk"] = dk_full.reshape(B, Hkv, G, S, D).sum(dim=2)
        res["dv"] = dv_full.reshape(B, Hkv, G, S, D).sum(dim=2)
    return res


def attention_rows(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, doc_ids: torch.Tensor,
                   dout: torch.Tensor, rows: list[torch.Tensor], *,
                   dtype: torch.dtype = torch.float64) -> dict[str, list[torch.Tensor]]:
    """``attention`` (flex semantics, default scale) at chosen query rows only.

    rows[b] = query positions of pack b.  Out, lse and dQ of a query row depend
    only on that row (its keys are the same-document positions <= it), so
    they are computed row by row, with no S x S work: out[b] [Hq, n, D],
    lse[b] [Hq, n], dq[b] [Hq, n, D] for the n rows of pack b, in ``dtype``.
    """
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    sc = 1.0 / math.sqrt(D)
    docs = doc_ids.detach().to("cpu", torch.int64).reshape(B, S)
    res: dict[str, list[torch.Tensor]] = {"out": [], "lse": [], "dq": []}
    for b in range(B):
        r = rows[b].to(torch.int64)
        # query head h = c * G + g reads KV head c
        Q = q[b].detach()[:, r.to(q.device)].to("cpu", dtype).view(Hkv, G, len(r), D)
        dO = dout[b].detach()[:, r.to(q.device)].to("cpu", dtype).view(Hkv, G, len(r), D)
        K = k[b].detach().to("cpu", dtype)
        V = v[b].detach().to("cpu", dtype)
        out = torch.zeros(Hkv, G, len(r), D, dtype=dtype)
        lse = torch.full((Hkv, G, len(r)), -math.inf, dtype=dtype)
        dq = torch.zeros_like(out)
        for n, qi in enumerate(r.tolist()):
            keys = torch.nonzero(docs[b, : qi + 1] == docs[b, qi]).flatten()
            Kk, Vk = K[:, keys], V[:, keys]
            s = torch.einsum("cgd,ckd->cgk", Q[:, :, n], Kk) * sc
            lse[:, :, n] = torch.logsumexp(s, dim=-1)
            p = torch.exp(s - lse[:, :, n, None])
            o = torch.einsum("cgk,ckd->cgd", p, Vk)
            out[:, :, n] = o
            dp = torch.einsum("cgd,ckd->cgk", dO[:, :, n], Vk)
            ds = p * (dp - (dO[:, :, n] * o).sum(-1, keepdim=True))
            dq[:, :, n] = torch.einsum("cgk,ckd->cgd", ds, Kk) * sc
        res["out"].append(out.reshape(Hq, len(r), D))
        res["lse"].append(lse.reshape(Hq, len(r)))
        res["dq"].append(dq.reshape(Hq, len(r), D))
    return res


def dense_mask(doc_ids: torch.Tensor) -> torch.Tensor:
    """[B, S, S] bool mask of attention.py:43-44 (for the SDPA cross-check)."""
    d = doc_ids.to(torch.int64)
    S = d.shape[-1]
    causal = torch.tril(torch.ones(S, S, dtype=torch.bool))
    return (d[:, :, None] == d[:, None, :]) & causal


def attention_flops(doc_lengths: list[int], head_dim: int, n_q_heads: int) -> dict[str, float]:
    """Algorithmic FLOPs of masked attention: fwd 4*D*Hq*P, bwd 8*D*Hq*P.

    P = sum over documents of L(L+1)/2 allowed (q, kv) pairs (causal within a
    document) -- the counting of the reference's cost model
    (``packbalance/data/cost.py:91-94,125-127``: train = 3 x forward).
    """
    pairs = float(sum(L * (L + 1) // 2 for L in doc_lengths))
    return {"pairs": pairs, "fwd": 4.0 * head_dim * n_q_heads * pairs,
            "bwd": 8.0 * head_dim * n_q_heads * pairs}
