"""Document-masked GQA attention over packed sequences on gfx950.

Drop-in for the reference ``packbalance/model/attention.py``:

* ``build_doc_block_mask(doc_ids, n_heads, block_size=128)`` (attention.py:25-54)
  returns a ``torch.nn.attention.flex_attention.BlockMask`` whose eight tables
  are bit-identical to ``create_block_mask``'s for the mask
  ``doc[q] == doc[kv] and q >= kv``, but are built by two small HIP kernels
  straight from ``doc_ids`` -- the dense [H, S, S] mask the reference
  materialises is never formed.  The returned object also carries ``doc_ids``
  and the attention kernel's own tile plan.
* ``attention_forward(q, k, v, doc_ids, *, block_mask=None, backend="auto",
  compile_attention=True)`` (attention.py:98-125) runs the hand-written MFMA
  kernels for ``backend`` "auto" / "flex"; ``compile_attention`` is accepted
  and ignored (nothing is traced or compiled at run time).
* ``DocPlans(doc_ids)`` is the mask as the native kernels consume it -- their
  tile plans, built on first use and cached -- for any batch of packs and
  without the FlexAttention tables (a training step that never hands its mask
  to FlexAttention has no reader for them).

This module has one path, the native one: CPU tensors, and ``backend="eager"``
(the reference's own per-document SDPA loop, ``eager_attention`` at
attention.py:66-95, which stays in the reference module), raise here.  The
reference-side binding keeps its own ``x.is_cuda`` dispatch, so CPU callers
still reach ``eager_attention`` there.
"""

from __future__ import annotations

import ctypes

import torch

from packbalance_amd import _native as N

try:
    from torch.nn.attention.flex_attention import BlockMask as _TorchBlockMask

    HAS_FLEX = True
except ImportError:  # pragma: no cover - torch without FlexAttention
    _TorchBlockMask = object
    HAS_FLEX = False

HAS_NATIVE = N.available()


def _block_size(seq_len: int, block_size: int) -> int:
    # attention.py:40-41: never below 32, a power of two, at most block_size.
    power_of_two = 1 << max(0, seq_len - 1).bit_length()
    return min(block_size, max(32, power_of_two))


class DocBlockMask(_TorchBlockMask):
    """A FlexAttention ``BlockMask`` for the document mask, plus ``doc_ids``.

    ``doc_ids`` is the int64 [B, S] tensor the tables were built from; the
    native attention reads it for the element mask of PARTIAL tiles.
    """

    def __init__(self, *args, doc_ids: torch.Tensor, **kwargs):
        super().__init__(*args, **kwargs)
        self.doc_ids = doc_ids
        self._plans: dict = {}


def doc_block_tables(doc_ids: torch.Tensor, n_heads: int, block: int) -> dict[str, torch.Tensor]:
    """The eight int32 BlockMask tables for doc_ids [B, S] (any B), on its device."""
    N.require_device(doc_ids, op="build_doc_block_mask")
    ids = doc_ids.to(torch.int64)
    if ids.dim() == 1:
        ids = ids[None]
    if ids.stride(-1) != 1:
        ids = ids.contiguous()
    b, s = ids.shape
    nblk = -(-s // block)
    dev = ids.device
    i32 = dict(dtype=torch.int32, device=dev)
    t = {
        "kv_num_blocks": torch.empty((b, n_heads, nblk), **i32),
        "kv_indices": torch.empty((b, n_heads, nblk, nblk), **i32),
        "full_kv_num_blocks": torch.empty((b, n_heads, nblk), **i32),
        "full_kv_indices": torch.empty((b, n_heads, nblk, nblk), **i32),
        "q_num_blocks": torch.empty((b, n_heads, nblk), **i32),
        "q_indices": torch.empty((b, n_heads, nblk, nblk), **i32),
        "full_q_num_blocks": torch.empty((b, n_heads, nblk), **i32),
        "full_q_indices": torch.empty((b, n_heads, nblk, nblk), **i32),
    }
    ws = torch.empty(b * nblk * nblk, dtype=torch.uint8, device=dev)
    N.call(
        "pb_doc_block_tables",
        ids.data_ptr(), ids.stride(0), b, s, block, n_heads,
        t["kv_num_blocks"].data_ptr(), t["kv_indices"].data_ptr(),
        t["full_kv_num_blocks"].data_ptr(), t["full_kv_indices"].data_ptr(),
        t["q_num_blocks"].data_ptr(), t["q_indices"].data_ptr(),
        t["full_q_num_blocks"].data_ptr(), t["full_q_indices"].data_ptr(),
        ws.data_ptr(), N.stream_ptr(ids),
    )
    return t


def build_doc_block_mask(doc_ids: torch.Tensor, n_heads: int, block_size: int = 128):
    """Build a BlockMask allowing causal attention inside each document.

    Same contract as the reference (attention.py:25-54): ``doc_ids`` is [S] or
    [1, S]; B > 1 raises ValueError; BLOCK = min(block_size, max(32, next_pow2(S))).
    """
    if doc_ids.dim() == 2:
        if doc_ids.shape[0] != 1:
            raise ValueError("build_doc_block_mask expects a single packed sequence")
    elif doc_ids.dim() != 1:
        raise ValueError("doc_ids must be [S] or [1, S]")
    seq_len = doc_ids.shape[-1]
    block = _block_size(seq_len, block_size)
    ids = doc_ids.reshape(1, seq_len).to(torch.int64)
    t = doc_block_tables(ids, n_heads, block)

    def mask_mod(b, h, q_idx, kv_idx):
        d = ids[0]
        return (d[q_idx] == d[kv_idx]) & (q_idx >= kv_idx)

    return DocBlockMask(
        (seq_len, seq_len),
        t["kv_num_blocks"], t["kv_indices"], t["full_kv_num_blocks"], t["full_kv_indices"],
        t["q_num_blocks"], t["q_indices"], t["full_q_num_blocks"], t["full_q_indices"],
        (block, block), mask_mod, doc_ids=ids,
    )


class DocPlans:
    """The document mask of ``doc_ids`` [B, S] (any B) for the native kernels only:
    holds the int64 doc ids and caches the kernels' tile plans per head shape."""

    def __init__(self, doc_ids: torch.Tensor) -> None:
        N.require_device(doc_ids, op="DocPlans")
        d = doc_ids.to(torch.int64)
        if d.dim() == 1:
            d = d[None]
        if d.dim() != 2:
            raise ValueError("doc_ids must be [S] or [B, S]")
        self.doc_ids = d.contiguous()
        self._plans: dict = {}


# ---------------------------------------------------------------- native attention
FWD, BWD_KV, BWD_Q = 0, 1, 2


def attn_config(b: int, hq: int, hkv: int, s: int, d: int) -> dict:
    """Tile sizes / workspace the kernels use for this shape (``pb_attn_config``)."""
    out = (ctypes.c_int64 * 10)()
    N.call("pb_attn_config", b, hq, hkv, s, d, out)
    return {"tiles": {FWD: (out[0], out[1]), BWD_KV: (out[2], out[3]), BWD_Q: (out[4], out[5])},
            "workspace": int(out[6]), "split": bool(out[7]), "fwd_workspace": int(out[8]),
            "fwd_chunk": int(out[9])}


class _Plan:
    """Tile plan of a packed batch for one kernel (see ``pb_attn_plan``)."""

    def __init__(self, doc: torch.Tensor, kernel: int, q_tile: int, kv_tile: int):
        self.q_tile, self.kv_tile = q_tile, kv_tile
        by_kv = 1 if kernel == BWD_KV else 0
        b, s = doc.shape
        nq = -(-s // self.q_tile)
        nk = -(-s // self.kv_tile)
        rows, cols = (nk, nq) if by_kv else (nq, nk)
        dev = doc.device
        self.counts = torch.empty((b, rows), dtype=torch.int32, device=dev)
        self.lists = torch.empty((b, rows, cols), dtype=torch.int32, device=dev)
        ws = torch.empty(b * nq * nk, dtype=torch.uint8, device=dev)
        N.call("pb_attn_plan", doc.data_ptr(), doc.stride(0), b, s, self.q_tile, self.kv_tile,
               by_kv, self.counts.data_ptr(), self.lists.data_ptr(), ws.data_ptr(),
               N.stream_ptr(doc))


def _doc_2d(doc_ids: torch.Tensor, batch: int, seq_len: int) -> torch.Tensor:
    d = doc_ids.to(torch.int64)
    if d.dim() == 1:
        d = d[None]
    if d.shape[-1] != seq_len or d.shape[0] not in (1, batch):
        raise ValueError(f"doc_ids shape {tuple(doc_ids.shape)} does not match [B={batch}, S={seq_len}]")
    if d.shape[0] != batch:
        d = d.expand(batch, seq_len)
    return d.contiguous()


def _plans(doc: torch.Tensor, hq: int, hkv: int, head_dim: int, block_mask) -> dict:
    """Plans for the three kernels; cached on a DocBlockMask built from the same doc_ids."""
    # The model passes the very doc_ids tensor the mask was built from; the
    # mask keeps it alive, so pointer identity is a sync-free cache key.
    cache = None
    if (isinstance(block_mask, (DocBlockMask, DocPlans)) and block_mask.doc_ids.shape == doc.shape
            and block_mask.doc_ids.data_ptr() == doc.data_ptr()):
        cache = block_mask._plans
    key = ("plans", hq, hkv, head_dim)
    if cache is not None and key in cache:
        return cache[key]
    b, s = doc.shape
    cfg = attn_config(b, hq, hkv, s, head_dim)
    plans = {k: _Plan(doc, k, *cfg["tiles"][k]) for k in (FWD, BWD_KV, BWD_Q)}
    plans["workspace"] = cfg["workspace"]
    plans["fwd_workspace"] = cfg["fwd_workspace"]
    if cache is not None:
        cache[key] = plans
    return plans


class _DocAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, doc, plans, scale, out_mem, dv_mem):
        B, Hq, S, D = q.shape
        Hkv = k.shape[1]
        if out_mem is None:
            out_mem = torch.empty((B, S, Hq, D), dtype=q.dtype, device=q.device)
        out = out_mem.transpose(1, 2)
        lse = torch.empty((B, Hq, S), dtype=torch.float32, device=q.device)
        p = plans[FWD]
        ws = None
        if plans["fwd_workspace"]:
            ws = torch.empty(plans["fwd_workspace"], dtype=torch.uint8, device=q.device)
        N.call("pb_attn_fwd", N.BHSD.of(q), N.BHSD.of(k), N.BHSD.of(v), N.BHSD.of(out),
               lse.data_ptr(), N.ptr(ws), doc.data_ptr(), doc.stride(0), p.counts.data_ptr(),
               p.lists.data_ptr(), B, Hq, Hkv, S, D, float(scale), N.PB_BF16, N.stream_ptr(q))
        ctx.save_for_backward(q, k, v, out, lse, doc)
        ctx.plans = plans
        ctx.scale = scale
        ctx.dv_mem = dv_mem
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse, doc = ctx.saved_tensors
        B, Hq, S, D = q.shape
        Hkv = k.shape[1]
        g = dout.to(torch.bfloat16)
        if g.stride(-1) != 1:
            g = g.contiguous()
        dq = torch.empty((B, S, Hq, D), dtype=q.dtype, device=q.device).transpose(1, 2)
        dk = torch.empty((B, S, Hkv, D), dtype=k.dtype, device=k.device).transpose(1, 2)
        if ctx.dv_mem is not None:  # the caller's [B, S, Hkv, D] view (e.g. a gradient slot)
            dv = ctx.dv_mem.transpose(1, 2)
        else:
            dv = torch.empty((B, S, Hkv, D), dtype=v.dtype, device=v.device).transpose(1, 2)
        ws = torch.empty(ctx.plans["workspace"], dtype=torch.uint8, device=q.device)
        pq, pkv = ctx.plans[BWD_Q], ctx.plans[BWD_KV]
        N.call("pb_attn_bwd", N.BHSD.of(q), N.BHSD.of(k), N.BHSD.of(v), N.BHSD.of(out),
               N.BHSD.of(g), N.BHSD.of(dq), N.BHSD.of(dk), N.BHSD.of(dv), lse.data_ptr(),
               ws.data_ptr(), doc.data_ptr(), doc.stride(0), pq.counts.data_ptr(),
               pq.lists.data_ptr(), pkv.counts.data_ptr(), pkv.lists.data_ptr(),
               B, Hq, Hkv, S, D, float(ctx.scale), N.PB_BF16, N.stream_ptr(q))
        return dq, dk, dv, None, None, None, None, None


class _DocAttentionF32(torch.autograd.Function):
    """fp32 q/k/v (the reference's non-autocast FlexAttention computes in fp32)."""

    @staticmethod
    def forward(ctx, q, k, v, doc, scale):
        B, Hq, S, D = q.shape
        Hkv = k.shape[1]
        out = torch.empty((B, S, Hq, D), dtype=torch.float32, device=q.device).transpose(1, 2)
        lse = torch.empty((B, Hq, S), dtype=torch.float32, device=q.device)
        N.call("pb_attn_fwd_f32", N.BHSD.of(q), N.BHSD.of(k), N.BHSD.of(v), N.BHSD.of(out),
               lse.data_ptr(), doc.data_ptr(), doc.stride(0), B, Hq, Hkv, S, D, float(scale),
               N.stream_ptr(q))
        ctx.save_for_backward(q, k, v, out, lse, doc)
        ctx.scale = scale
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse, doc = ctx.saved_tensors
        B, Hq, S, D = q.shape
        Hkv = k.shape[1]
        g = _bhsd(dout.to(torch.float32))
        dq = torch.empty((B, S, Hq, D), dtype=torch.float32, device=q.device).transpose(1, 2)
        dk = torch.empty((B, S, Hkv, D), dtype=torch.float32, device=q.device).transpose(1, 2)
        dv = torch.empty((B, S, Hkv, D), dtype=torch.float32, device=q.device).transpose(1, 2)
        ws = torch.empty(N.lib().pb_attn_bwd_f32_workspace_bytes(B, Hq, Hkv, S, D),
                         dtype=torch.uint8, device=q.device)
        N.call("pb_attn_bwd_f32", N.BHSD.of(q), N.BHSD.of(k), N.BHSD.of(v), N.BHSD.of(out),
               N.BHSD.of(g), N.BHSD.of(dq), N.BHSD.of(dk), N.BHSD.of(dv), lse.data_ptr(),
               ws.data_ptr(), doc.data_ptr(), doc.stride(0), B, Hq, Hkv, S, D,
               float(ctx.scale), N.stream_ptr(q))
        return dq, dk, dv, None, None


def _bhsd(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def doc_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, doc_ids: torch.Tensor,
                  *, block_mask=None, scale: float | None = None,
                  out: torch.Tensor | None = None,
                  dv_out: torch.Tensor | None = None) -> torch.Tensor:
    """Document-masked causal GQA attention on the gfx950 kernels.

    q [B, Hq, S, D], k/v [B, Hkv, S, D] (any strides with unit D stride),
    doc_ids [B, S] or [S].  bf16 q/k/v run the MFMA kernels (bf16 operands,
    fp32 accumulation); fp32 (and fp16, widened) run the fp32 kernels, as the
    reference's FlexAttention computes fp32 tensors in fp32; the result has
    q's dtype.  Returns [B, Hq, S, D] (a transposed view of [B, S, Hq, D] memory;
    with ``out``, a contiguous bf16 [B, S, Hq, D] buffer for bf16 inputs, that
    buffer).  ``dv_out`` (bf16 inputs): a bf16 [B, S, Hkv, D] view with unit D
    stride (e.g. columns of a fused qkv gradient) that the backward writes dV
    into and returns (transposed) as v's gradient.
    """
    N.require_device(q, k, v, doc_ids, op="attention_forward")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be [B, H, S, D]")
    B, Hq, S, D = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[2] != S or k.shape[3] != D:
        raise ValueError(f"k {tuple(k.shape)} / v {tuple(v.shape)} do not match q {tuple(q.shape)}")
    if Hq % k.shape[1]:
        raise ValueError("query heads must be a multiple of key/value heads")
    if D > 128:
        raise RuntimeError(f"head_dim {D} > 128 is not supported by the attention kernels")
    doc = _doc_2d(doc_ids, B, S)
    sc = (1.0 / D ** 0.5) if scale is None else float(scale)
    dtype = q.dtype
    if out is not None and (dtype != torch.bfloat16 or out.dtype != torch.bfloat16
                            or out.shape != (B, S, Hq, D) or not out.is_contiguous()):
        raise ValueError("doc_attention: out must be a contiguous bf16 [B, S, Hq, D] tensor "
                         "(bf16 inputs)")
    if dv_out is not None and (dtype != torch.bfloat16 or dv_out.dtype != torch.bfloat16
                               or dv_out.shape != (B, S, k.shape[1], D)
                               or dv_out.stride(-1) != 1):
        raise ValueError("doc_attention: dv_out must be a bf16 [B, S, Hkv, D] view with unit "
                         "D stride (bf16 inputs)")
    if dtype != torch.bfloat16:
        qf, kf, vf = (_bhsd(t.to(torch.float32)) for t in (q, k, v))
        o = _DocAttentionF32.apply(qf, kf, vf, doc, sc)
        return o if dtype == torch.float32 else o.to(dtype)
    plans = _plans(doc, Hq, k.shape[1], D, block_mask)
    qb, kb, vb = (_bhsd(t.to(torch.bfloat16)) for t in (q, k, v))
    return _DocAttention.apply(qb, kb, vb, doc, plans, sc, out, dv_out)


def flex_attention(query, key, value, block_mask=None, enable_gqa: bool = False, scale=None):
    """FlexAttention-style entry for the document mask (reference test calling convention).

    ``block_mask`` must be a mask from :func:`build_doc_block_mask`; its doc_ids
    define the mask.
    """
    if not isinstance(block_mask, DocBlockMask):
        raise ValueError("flex_attention here needs the BlockMask of build_doc_block_mask")
    if query.shape[1] != key.shape[1] and not enable_gqa:
        raise ValueError("query and key heads differ; pass enable_gqa=True")
    return doc_attention(query, key, value, block_mask.doc_ids, block_mask=block_mask, scale=scale)


def attention_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, doc_ids: torch.Tensor,
                      *, block_mask=None, backend: str = "auto",
                      compile_attention: bool = True) -> torch.Tensor:
    """The flex branch of the reference dispatch (attention.py:98-125) on the native kernels.

    "auto" and "flex" run the gfx950 kernels on device tensors (CPU tensors
    raise RuntimeError).  "eager" is the reference's own ``eager_attention``,
    which is not part of this package: RuntimeError.  Anything else raises
    ValueError, as in the reference.  ``compile_attention`` is accepted for API
    compatibility (nothing is compiled at run time).
    """
    del compile_attention
    if backend in ("auto", "flex"):
        return doc_attention(q, k, v, doc_ids, block_mask=block_mask)
    if backend == "eager":
        raise RuntimeError("attention_forward(backend='eager') is the reference's eager_attention "
                           "(packbalance/model/attention.py:66-95); packbalance_amd runs only the "
                           "native kernels")
    raise ValueError(f"unknown attention backend {backend}")
