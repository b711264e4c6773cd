"""Minimal Llama-style decoder that drives the hot path (benchmark harness).

It exercises the hot-path calls exactly where the reference model makes them
(``packbalance/model/llama.py``): RMSNorm at :43-46, SwiGLU at :57-61,
attention at :77-103 (q/k/v as ``.transpose(1, 2)`` views of [B, S, H, D]),
the block mask at :147-152 and the summed linear CE at :222-242, with the same
dtype flow under ``torch.autocast(bf16)`` (fp32 embeddings and residual
stream, bf16 projections, fp32 tied LM head).  Weights are random
(``init_std`` normal, residual projections scaled by 1/sqrt(2 n_layers) as at
:191-201).

``forward`` is the training path: parameters live in one flat fp32 store
(``FlatParams``) with a compute-dtype copy, q/k/v and gate/up are single
GEMMs against stacked weights, every residual add is fused into the next
RMSNorm (which writes the compute dtype directly: no autocast casts), and
weight gradients accumulate in fp32 inside the backward GEMMs.  Its math is
the reference's with fewer roundings (dW and the fused input gradients are
never rounded to bf16).  ``forward_unfused`` is the module-by-module form
under autocast, kept for comparison.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import nn

from packbalance_amd.kernels.fused_ce import (
    linear_cross_entropy,
    linear_cross_entropy_accumulate,
    lmhead_weight_bf16,
)
from packbalance_amd.kernels.rmsnorm import add_rmsnorm, rmsnorm, rmsnorm_to
from packbalance_amd.kernels.swiglu import swiglu
from packbalance_amd.model import layers as L
from packbalance_amd.model.attention import attention_forward, build_doc_block_mask, doc_attention
from packbalance_amd.model.flat import FlatParams
from packbalance_amd.model.rope import RotaryEmbedding, apply_rotary_pos_emb


@dataclass
class ModelConfig:
    """The model fields of the reference ``packbalance/config.py:15-55``."""

    vocab_size: int = 32000
    d_model: int = 768
    n_layers: int = 12
    n_heads: int = 12
    n_kv_heads: int = 4
    d_ff: int = 2048
    max_seq_len: int = 2048
    rope_theta: float = 10000.0
    norm_eps: float = 1e-5
    tie_embeddings: bool = True
    attention_backend: str = "auto"
    ce_chunk_size: int = 1024
    z_loss_coeff: float = 0.0
    init_std: float = 0.02

    def __post_init__(self) -> None:
        if self.d_model % self.n_heads:
            raise ValueError("d_model must be divisible by n_heads")
        if self.n_heads % self.n_kv_heads:
            raise ValueError("n_heads must be divisible by n_kv_heads")

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads


def cfg1_model() -> ModelConfig:
    return ModelConfig(vocab_size=512, d_model=128, n_layers=2, n_heads=4, n_kv_heads=2,
                       d_ff=344, max_seq_len=256)


def cfg2_model() -> ModelConfig:
    return ModelConfig()


class RMSNorm(nn.Module):
    def __init__(self, d_model: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d_model))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rmsnorm(x, self.weight, self.eps)


class LlamaMLP(nn.Module):
    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.gate_proj = nn.Linear(cfg.d_model, cfg.d_ff, bias=False)
        self.up_proj = nn.Linear(cfg.d_model, cfg.d_ff, bias=False)
        self.down_proj = nn.Linear(cfg.d_ff, cfg.d_model, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(swiglu(self.gate_proj(x), self.up_proj(x)))

    def groups(self):
        return {"gu": [self.gate_proj.weight, self.up_proj.weight], "down": [self.down_proj.weight]}

    def fused(self, x: torch.Tensor, flat: FlatParams, dt: torch.dtype, wt: dict,
              plan: L.WgradPlan | None = None, layer: int | None = None) -> torch.Tensor:
        gr = self.groups()
        a = L.gate_up_swiglu(x, flat.weight(gr["gu"], dt), flat.grad_of(gr["gu"]), wt["gu"],
                             plan, layer)
        return L.linear(a, flat.weight(gr["down"], dt), flat.grad_of(gr["down"]), wt["down"],
                        plan, "down", layer)


class LlamaAttention(nn.Module):
    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.n_heads, self.n_kv_heads, self.head_dim = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        self.q_proj = nn.Linear(cfg.d_model, cfg.n_heads * cfg.head_dim, bias=False)
        self.k_proj = nn.Linear(cfg.d_model, cfg.n_kv_heads * cfg.head_dim, bias=False)
        self.v_proj = nn.Linear(cfg.d_model, cfg.n_kv_heads * cfg.head_dim, bias=False)
        self.o_proj = nn.Linear(cfg.n_heads * cfg.head_dim, cfg.d_model, bias=False)
        self.backend = cfg.attention_backend

    def forward(self, hidden, cos, sin, doc_ids, block_mask=None):
        b, s, _ = hidden.shape
        q = self.q_proj(hidden).view(b, s, self.n_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(hidden).view(b, s, self.n_kv_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(hidden).view(b, s, self.n_kv_heads, self.head_dim).transpose(1, 2)
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        out = attention_forward(q, k, v, doc_ids, block_mask=block_mask, backend=self.backend)
        return self.o_proj(out.transpose(1, 2).contiguous().view(b, s, -1))

    def groups(self):
        return {"qkv": [self.q_proj.weight, self.k_proj.weight, self.v_proj.weight],
                "o": [self.o_proj.weight]}

    def fused(self, x, cos, sin, doc_ids, block_mask, flat: FlatParams, dt: torch.dtype,
              wt: dict, plan: L.WgradPlan | None = None, layer: int | None = None):
        b, s, _ = x.shape
        gr = self.groups()
        q, k, v = L.qkv_rope(x, flat.weight(gr["qkv"], dt), flat.grad_of(gr["qkv"]), cos, sin,
                             self.n_heads, self.n_kv_heads, self.head_dim, wt["qkv"], plan, layer)
        if plan is not None and self.backend in ("auto", "flex") and q.dtype == torch.bfloat16:
            # the attention output lands in the o projection's input slot, and dV in the
            # v columns of the qkv projection's gradient slot
            nqk = (self.n_heads + self.n_kv_heads) * self.head_dim
            out = doc_attention(q, k, v, doc_ids, block_mask=block_mask,
                                out=plan.x_of("o", layer).view(b, s, self.n_heads, self.head_dim),
                                dv_out=plan.dy_of("qkv", layer)[:, nqk:].view(
                                    b, s, self.n_kv_heads, self.head_dim))
        else:
            out = attention_forward(q, k, v, doc_ids, block_mask=block_mask, backend=self.backend)
        o = out.transpose(1, 2).reshape(b, s, -1)
        return L.linear(o, flat.weight(gr["o"], dt), flat.grad_of(gr["o"]), wt["o"], plan, "o",
                        layer)


class LlamaDecoderLayer(nn.Module):
    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.self_attn = LlamaAttention(cfg)
        self.post_attention_layernorm = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.mlp = LlamaMLP(cfg)

    def forward(self, hidden, cos, sin, doc_ids, block_mask=None):
        hidden = hidden + self.self_attn(self.input_layernorm(hidden), cos, sin, doc_ids, block_mask)
        return hidden + self.mlp(self.post_attention_layernorm(hidden))

    def fused(self, hidden, pending, cos, sin, doc_ids, block_mask, flat: FlatParams,
              dt: torch.dtype, wt: dict, plan: L.WgradPlan | None = None,
              layer: int | None = None):
        """(new residual, MLP output still to be added): the previous layer's MLP
        output ``pending`` is added inside this layer's first norm.  With a
        weight-gradient ``plan``, the norms write the projections' inputs and the
        gradients of the added sublayer outputs straight into its slots."""
        eps = self.input_layernorm.eps
        w1, w2 = self.input_layernorm.weight, self.post_attention_layernorm.weight
        none = lambda kind, i: None  # noqa: E731
        x_slot = none if plan is None else plan.x_of
        dy_slot = none if plan is None else plan.dy_of
        # Norm weight gradients: reduced by the plan at the end of the backward
        # (norm slots 2 layer and 2 layer + 1; the final norm takes 2 L).
        defer = (lambda i: None) if plan is None else (lambda i: (plan, i))  # noqa: E731
        if pending is None:
            x = rmsnorm_to(hidden, w1, eps, dt, dw_acc=flat.grad_of([w1]),
                           y_out=x_slot("qkv", layer), dw_defer=defer(2 * layer))
        else:
            hidden, x = add_rmsnorm(hidden, pending, w1, eps, dt, dw_acc=flat.grad_of([w1]),
                                    y_out=x_slot("qkv", layer),
                                    ddelta_out=dy_slot("down", layer - 1),
                                    dw_defer=defer(2 * layer))
        a = self.self_attn.fused(x, cos, sin, doc_ids, block_mask, flat, dt, wt, plan, layer)
        hidden, x = add_rmsnorm(hidden, a, w2, eps, dt, dw_acc=flat.grad_of([w2]),
                                y_out=x_slot("gate_up", layer), ddelta_out=dy_slot("o", layer),
                                dw_defer=defer(2 * layer + 1))
        return hidden, self.mlp.fused(x, flat, dt, wt, plan, layer)


class LlamaForCausalLM(nn.Module):
    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.cfg = cfg
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.layers = nn.ModuleList([LlamaDecoderLayer(cfg) for _ in range(cfg.n_layers)])
        self.norm = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.rotary = RotaryEmbedding(cfg.head_dim, cfg.max_seq_len, cfg.rope_theta)
        for m in self.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                nn.init.normal_(m.weight, mean=0.0, std=cfg.init_std)
        scale = 1.0 / math.sqrt(2 * cfg.n_layers)
        for layer in self.layers:
            nn.init.normal_(layer.self_attn.o_proj.weight, mean=0.0, std=cfg.init_std * scale)
            nn.init.normal_(layer.mlp.down_proj.weight, mean=0.0, std=cfg.init_std * scale)
        self._flat: FlatParams | None = None
        self._lm_bf16 = None  # (compute copy, its refresh count, wb, wt) of the tied LM head

    # ------------------------------------------------------------ flat storage
    def flat_parameters(self, grad_slots: int = 1) -> FlatParams:
        """The flat store of this model's parameters (created on first use, and again
        if the parameters were moved or replaced since, or more gradient slots are
        asked for than it has)."""
        if (self._flat is None or not self._flat.owns(self)
                or self._flat.grad_slots < grad_slots):
            groups = []
            for layer in self.layers:
                a, m = layer.self_attn, layer.mlp
                groups.append([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight])
                groups.append([m.gate_proj.weight, m.up_proj.weight])
            self._flat = FlatParams(self, groups, grad_slots)
            self._lm_bf16 = None
        return self._flat

    def _lm_head(self, flat: FlatParams, dt: torch.dtype):
        """bf16 LM-head rows and their transpose, rebuilt whenever the compute copy was."""
        w = flat.weight([self.embed_tokens.weight], dt)
        c = self._lm_bf16
        if c is None or c[0] is not w or c[1] != flat.refreshes:
            self._lm_bf16 = c = (w, flat.refreshes) + lmhead_weight_bf16(w)
        return c[2], c[3]

    def _transposed_weights(self, flat: FlatParams, dt: torch.dtype) -> dict:
        """Every layer's projection weights transposed, one copy per kind (the
        input-gradient GEMMs read them)."""
        kinds = {}
        for layer in self.layers:
            for k, g in {**layer.self_attn.groups(), **layer.mlp.groups()}.items():
                kinds.setdefault(k, []).append(g)
        return {k: flat.transposed(g, dt) for k, g in kinds.items()}

    def _wgrad_plan(self, tokens: int, dt: torch.dtype, dev: torch.device):
        """The batched weight-gradient plan of one training forward (None when no
        backward can follow -- grad mode off or no parameter requiring grad --,
        in fp32, or when ``L.WGRAD_BATCHED`` is off)."""
        if (not L.WGRAD_BATCHED or dt == torch.float32 or dev.type != "cuda"
                or not torch.is_grad_enabled() or len(self.layers) < 2
                or not any(p.requires_grad for p in self.parameters())):
            return None
        c = self.cfg
        nq, nkv = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
        dims = {"qkv": (nq + 2 * nkv, c.d_model), "o": (c.d_model, nq),
                "gate_up": (2 * c.d_ff, c.d_model), "down": (c.d_model, c.d_ff)}
        return L.WgradPlan(len(self.layers), tokens, dims, dt, dev,
                           norms=2 * len(self.layers) + 1, norm_dim=c.d_model)

    def prepare(self, dt: torch.dtype) -> None:
        """Build the weight copies that forwards share (compute copy, transposed
        weights, LM-head rows) on the current stream.  Forwards run concurrently
        on other streams after it only read them (their stream waits for this
        one first); inside ``FlatParams.hold`` they are not rebuilt."""
        flat = self.flat_parameters()
        flat.refresh(dt)
        if dt != torch.float32:
            self._transposed_weights(flat, dt)
            if self.cfg.d_model % 8 == 0:
                self._lm_head(flat, dt)

    def forward(self, input_ids, labels, position_ids, doc_ids, block_mask=None):
        dev = input_ids.device
        dt = torch.get_autocast_dtype(dev.type) if torch.is_autocast_enabled(dev.type) else torch.float32
        flat = self.flat_parameters()
        flat.attach_grads()
        flat.refresh(dt)
        with torch.autocast(dev.type, enabled=False):
            emb = [self.embed_tokens.weight]
            hidden = L.embed(input_ids, self.embed_tokens.weight, flat.grad_of(emb))
            cos, sin = self.rotary(position_ids)
            if block_mask is None:
                block_mask = build_doc_block_mask(doc_ids, self.cfg.n_heads)
            wts = self._transposed_weights(flat, dt)
            plan = self._wgrad_plan(input_ids.numel(), dt, dev)
            pending = None
            for i, layer in enumerate(self.layers):
                hidden, pending = layer.fused(hidden, pending, cos, sin, doc_ids, block_mask, flat,
                                              dt, {k: w[i] for k, w in wts.items()}, plan, i)
            _, y = add_rmsnorm(hidden, pending, self.norm.weight, self.norm.eps, dt,
                               dw_acc=flat.grad_of([self.norm.weight]),
                               ddelta_out=None if plan is None else plan.dy_of(
                                   "down", len(self.layers) - 1),
                               dw_defer=None if plan is None else (plan, 2 * len(self.layers)))
            kw = dict(ignore_index=-100, z_loss_coeff=self.cfg.z_loss_coeff)
            if dt == torch.float32 or self.cfg.d_model % 8:
                return linear_cross_entropy(y, self.embed_tokens.weight, labels,
                                            chunk_size=self.cfg.ce_chunk_size, **kw)
            wb, wt = self._lm_head(flat, dt)
            return linear_cross_entropy_accumulate(y, wb, wt, flat.grad_of(emb), labels, **kw)

    def forward_unfused(self, input_ids, labels, position_ids, doc_ids, block_mask=None):
        """Module-by-module forward (``nn.Linear`` under the caller's autocast)."""
        hidden = self.embed_tokens(input_ids)
        cos, sin = self.rotary(position_ids)
        if block_mask is None:
            block_mask = build_doc_block_mask(doc_ids, self.cfg.n_heads)
        for layer in self.layers:
            hidden = layer(hidden, cos, sin, doc_ids, block_mask)
        hidden = self.norm(hidden)
        return linear_cross_entropy(hidden, self.embed_tokens.weight, labels,
                                    chunk_size=self.cfg.ce_chunk_size, ignore_index=-100,
                                    z_loss_coeff=self.cfg.z_loss_coeff)


def count_parameters(model: nn.Module) -> int:
    return sum(p.numel() for p in model.parameters())
