"""CPU restatement of the reference model's eager path (test oracle and CPU baseline).

This is what ``packbalance/model/llama.py`` runs when tensors are on the CPU
(``llama.py:147-152`` skips the block mask; ``kernels/*.py`` fall back to
``kernels/reference.py``; attention takes ``eager_attention``,
``model/attention.py:66-95``; CE is ``chunked_linear_cross_entropy``,
``kernels/reference.py:20-48``), written with torch CPU autograd over the same
parameter names as ``packbalance_amd.model.llama.LlamaForCausalLM`` so both
can share one state dict.  Default dtype fp32 -- the reference's CPU dtype.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def _rmsnorm(x, w, eps):
    # kernels/reference.py:9-13
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps) * w.float()).to(x.dtype)


def _rope(q, k, position_ids, head_dim, theta):
    # model/rope.py:9-42 (fp32 cache, rotate_half)
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    freqs = position_ids.to(torch.float32)[..., None] * inv
    cos = torch.cat((freqs.cos(), freqs.cos()), dim=-1).unsqueeze(1).to(q.dtype)
    sin = torch.cat((freqs.sin(), freqs.sin()), dim=-1).unsqueeze(1).to(q.dtype)

    def rot(x):
        h = x.shape[-1] // 2
        return torch.cat((-x[..., h:], x[..., :h]), dim=-1)

    return q * cos + rot(q) * sin, k * cos + rot(k) * sin


def _eager_attention(q, k, v, doc_ids):
    # model/attention.py:66-95: per document id >= 0, causal SDPA; pad rows 0.
    b_, h, s, d = q.shape
    g = h // k.shape[1]
    if g > 1:
        k = k.repeat_interleave(g, dim=1)
        v = v.repeat_interleave(g, dim=1)
    out = torch.zeros_like(q)
    for b in range(b_):
        ids = doc_ids[b]
        for doc in torch.unique(ids).tolist():
            if doc < 0:
                continue
            idx = (ids == doc).nonzero(as_tuple=True)[0]
            out[b : b + 1, :, idx] = F.scaled_dot_product_attention(
                q[b : b + 1, :, idx], k[b : b + 1, :, idx], v[b : b + 1, :, idx], is_causal=True)
    return out


def _chunked_ce(x, w, targets, chunk_size, z):
    # kernels/reference.py:20-48
    x2d = x.reshape(-1, x.shape[-1])
    t1d = targets.reshape(-1)
    total = x2d.new_zeros(())
    for s in range(0, x2d.shape[0], chunk_size):
        logits = x2d[s : s + chunk_size] @ w.t()
        y = t1d[s : s + chunk_size]
        total = total + F.cross_entropy(logits, y, ignore_index=-100, reduction="sum")
        if z:
            lse = torch.logsumexp(logits.float(), dim=-1)
            total = total + z * (lse[y != -100] ** 2).sum()
    return total


def _attention(x, p, pre, cfg, position_ids, doc_ids):
    # llama.py:77-103: q/k/v projections, RoPE on q and k, document-masked
    # attention, heads back to [B, S, Hq * D], then o_proj.
    b, s, _ = x.shape
    hd = cfg.d_model // cfg.n_heads
    q = (x @ p[pre + "self_attn.q_proj.weight"].t()).view(b, s, cfg.n_heads, hd).transpose(1, 2)
    k = (x @ p[pre + "self_attn.k_proj.weight"].t()).view(b, s, cfg.n_kv_heads, hd).transpose(1, 2)
    v = (x @ p[pre + "self_attn.v_proj.weight"].t()).view(b, s, cfg.n_kv_heads, hd).transpose(1, 2)
    q, k = _rope(q, k, position_ids, hd, cfg.rope_theta)
    a = _eager_attention(q, k, v, doc_ids)
    return a.transpose(1, 2).reshape(b, s, -1) @ p[pre + "self_attn.o_proj.weight"].t()


def _mlp(x, p, pre):
    # llama.py:57-61: silu(gate_proj(x)) * up_proj(x), then down_proj.
    gate = x @ p[pre + "mlp.gate_proj.weight"].t()
    up = x @ p[pre + "mlp.up_proj.weight"].t()
    return (F.silu(gate) * up) @ p[pre + "mlp.down_proj.weight"].t()


def _layer(h, p, pre, cfg, position_ids, doc_ids):
    # llama.py:122-125: pre-norm residual blocks; the residual stream h is
    # carried un-normalised and each block's output is added to it.
    eps = cfg.norm_eps
    h = h + _attention(_rmsnorm(h, p[pre + "input_layernorm.weight"], eps), p, pre, cfg,
                       position_ids, doc_ids)
    return h + _mlp(_rmsnorm(h, p[pre + "post_attention_layernorm.weight"], eps), p, pre)


def loss(params: dict[str, torch.Tensor], cfg, input_ids, labels, position_ids, doc_ids):
    """Summed CE loss of one pack batch through the eager CPU path (differentiable)."""
    p = params
    h = F.embedding(input_ids, p["embed_tokens.weight"])
    for i in range(cfg.n_layers):
        h = _layer(h, p, f"layers.{i}.", cfg, position_ids, doc_ids)
    h = _rmsnorm(h, p["norm.weight"], cfg.norm_eps)
    return _chunked_ce(h, p["embed_tokens.weight"], labels, cfg.ce_chunk_size, cfg.z_loss_coeff)


def cpu_params(model: torch.nn.Module, dtype=torch.float32) -> dict[str, torch.Tensor]:
    """Leaf CPU copies of a model's parameters (requires_grad), keyed like its state dict."""
    return {n: t.detach().to("cpu", dtype).clone().requires_grad_(True)
            for n, t in model.named_parameters()}
