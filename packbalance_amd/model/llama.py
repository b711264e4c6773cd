"""Minimal Llama-style decoder that drives the hot path (benchmark harness).

It exercises the hot-path calls exactly where the reference model makes them
(``packbalance/model/llama.py``): RMSNorm at :43-46, SwiGLU at :57-61,
attention at :77-103 (q/k/v as ``.transpose(1, 2)`` views of [B, S, H, D]),
the block mask at :147-152 and the summed linear CE at :222-242, with the same
dtype flow under ``torch.autocast(bf16)`` (fp32 embeddings and residual
stream, bf16 projections, fp32 tied LM head).  Weights are random
(``init_std`` normal, residual projections scaled by 1/sqrt(2 n_layers) as at
:191-201).  Everything that is not a hot-path kernel (embedding, projections,
RoPE) is plain PyTorch.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import nn

from packbalance_amd.kernels.fused_ce import linear_cross_entropy
from packbalance_amd.kernels.rmsnorm import rmsnorm
from packbalance_amd.kernels.swiglu import swiglu
from packbalance_amd.model.attention import attention_forward, build_doc_block_mask
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

    def forward(self, input_ids, labels, position_ids, doc_ids, block_mask=None):
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
