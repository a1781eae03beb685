"""The decode step around the W4A16 projections: a Llama / Qwen3 dense decoder on libtandem_w4.so.

The model classes of python/tandem/models/llama_family.py (12vivi/tandem), cut to what a decode
step runs besides attention:

    DecoderConfig     the fields of config.json the step needs     python/tandem/model_config.py
    GatedMLP          gate_up (SwiGLU epilogue) + down             python/tandem/layers/mlp.py:16-45
    Attention         qkv_proj + o_proj around the attention       python/tandem/layers/attention.py
    DecoderLayer      add+norm, attention, add+norm, MLP with the  python/tandem/models/llama_family.py:35-67
                      residual stream carried between layers
    DecoderModel      embedding, layers, final add+norm, lm_head   python/tandem/models/llama_family.py:70-116

Attention over a KV cache (paged cache, FlashInfer, RoPE, QK-norm) is another path of tandem and is
not part of this build. ``Attention.attend`` computes attention over a one-token context, the
first decode position: softmax over a single key is 1, so each query head's output is the value row
of its KV head (grouped-query attention). That is exact for that position and costs one small copy
kernel, so a captured step has the real launch sequence of a decoder layer around the projections.

Projections are W4Linear (AutoAWQ checkpoints) or nn.Linear (fp16 checkpoints); ``prepare`` moves
the model to the GPU, repacks the W4 layers and routes the fp16 projections and the logits head
through layers/gemv16.py's table. Norms run on tw4_rms_norm / tw4_add_rms_norm, or inside the W4
qkv_proj / gate_up_proj kernels where W4Linear.forward_norm fuses them (the decode GEMV at the
batch sizes it runs: a norm kernel fewer before each, the same bits).
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Any, Optional

import torch
from torch import nn

from tandem_amd.layers import gemv16, norm
from tandem_amd.layers.linear import finalize_quantized, make_linear


@dataclass(frozen=True)
class DecoderConfig:
    hidden_size: int
    intermediate_size: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    num_layers: int
    vocab_size: int
    rms_norm_eps: float = 1e-6
    tie_word_embeddings: bool = False

    @classmethod
    def from_hf(cls, d: dict[str, Any]) -> "DecoderConfig":
        """The fields of a Hugging Face config.json (python/tandem/model_config.py)."""
        heads = int(d["num_attention_heads"])
        return cls(hidden_size=int(d["hidden_size"]), intermediate_size=int(d["intermediate_size"]),
                   num_heads=heads, num_kv_heads=int(d.get("num_key_value_heads", heads)),
                   head_dim=int(d.get("head_dim") or d["hidden_size"] // heads),
                   num_layers=int(d["num_hidden_layers"]), vocab_size=int(d["vocab_size"]),
                   rms_norm_eps=float(d.get("rms_norm_eps", 1e-6)),
                   tie_word_embeddings=bool(d.get("tie_word_embeddings", False)))


QWEN3_8B = DecoderConfig(4096, 12288, 32, 8, 128, 36, 151936)
QWEN3_1_7B = DecoderConfig(2048, 6144, 16, 8, 128, 28, 151936, tie_word_embeddings=True)


def silu_and_mul(y: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up on [..., gate | up] (the separate activation of an unfused MLP)."""
    half = y.shape[-1] // 2
    return torch.nn.functional.silu(y[..., :half]) * y[..., half:]


class GatedMLP(nn.Module):
    """SwiGLU MLP with one fused gate_up projection (python/tandem/layers/mlp.py:16-45): with an
    AWQ checkpoint the gate_up W4Linear applies SwiGLU in its kernel epilogue unless
    TANDEM_W4_FUSE_ACT=0."""

    def __init__(self, hidden_size: int, intermediate_size: int, quant: Optional[Any] = None) -> None:
        super().__init__()
        self.intermediate_size = intermediate_size
        self.gate_up_proj = make_linear(hidden_size, 2 * intermediate_size, False, quant)
        self.down_proj = make_linear(intermediate_size, hidden_size, False, quant)
        enable = getattr(self.gate_up_proj, "enable_silu_mul", None)
        self.fused_act = bool(enable is not None and os.environ.get("TANDEM_W4_FUSE_ACT", "1") != "0" and enable())

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.fused_act:
            return self.down_proj(self.gate_up_proj(x))
        return self.down_proj(silu_and_mul(self.gate_up_proj(x)))


class Attention(nn.Module):
    """The projections of grouped-query attention; ``attend`` is the one-token-context attention
    described in the module docstring."""

    def __init__(self, cfg: DecoderConfig, quant: Optional[Any] = None) -> None:
        super().__init__()
        self.num_heads, self.num_kv_heads, self.head_dim = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
        self.q_size = cfg.num_heads * cfg.head_dim
        self.kv_size = cfg.num_kv_heads * cfg.head_dim
        self.qkv_proj = make_linear(cfg.hidden_size, self.q_size + 2 * self.kv_size, False, quant)
        self.o_proj = make_linear(self.q_size, cfg.hidden_size, False, quant)

    def attend(self, qkv: torch.Tensor) -> torch.Tensor:
        """[M, q | k | v] -> [M, num_heads * head_dim]: query head h takes the value row of KV head
        h // (num_heads / num_kv_heads)."""
        m = qkv.shape[0]
        v = qkv[:, self.q_size + self.kv_size:].view(m, self.num_kv_heads, 1, self.head_dim)
        group = self.num_heads // self.num_kv_heads
        return v.expand(m, self.num_kv_heads, group, self.head_dim).reshape(m, self.q_size).contiguous()

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        return self.o_proj(self.attend(self.qkv_proj(hidden)))


class DecoderLayer(nn.Module):
    def __init__(self, cfg: DecoderConfig, quant: Optional[Any] = None) -> None:
        super().__init__()
        self.self_attn = Attention(cfg, quant)
        self.mlp = GatedMLP(cfg.hidden_size, cfg.intermediate_size, quant)
        self.input_layernorm = norm.RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.post_attention_layernorm = norm.RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)

    def forward(self, hidden: torch.Tensor, residual: Optional[torch.Tensor]) -> tuple[torch.Tensor, torch.Tensor]:
        """The residual stream is carried between layers, so every "add residual, then normalise"
        pair is one kernel (python/tandem/models/llama_family.py:47-67)."""
        n1, n2 = self.input_layernorm, self.post_attention_layernorm
        attn, mlp = self.self_attn, self.mlp
        if hasattr(attn.qkv_proj, "forward_norm"):  # W4: the norm goes into the projection's prologue
            qkv, residual = attn.qkv_proj.forward_norm(hidden, residual, n1.weight, n1.eps)
            hidden = attn.o_proj(attn.attend(qkv))
        else:
            if residual is None:
                residual = hidden
                hidden = norm.rms_norm(hidden, n1.weight, n1.eps)
            else:
                hidden, residual = norm.fused_add_rms_norm(hidden, residual, n1.weight, n1.eps)
            hidden = attn(hidden)
        if hasattr(mlp.gate_up_proj, "forward_norm"):
            act, residual = mlp.gate_up_proj.forward_norm(hidden, residual, n2.weight, n2.eps)
            return mlp.down_proj(act if mlp.fused_act else silu_and_mul(act)), residual
        hidden, residual = norm.fused_add_rms_norm(hidden, residual, n2.weight, n2.eps)
        return mlp(hidden), residual


class DecoderModel(nn.Module):
    """Parameter names follow the Hugging Face checkpoints (model.embed_tokens, model.layers.N.*,
    model.norm, lm_head) except the fused qkv_proj and gate_up_proj that tandem_amd.loader
    assembles."""

    def __init__(self, cfg: DecoderConfig, quant: Optional[Any] = None) -> None:
        super().__init__()
        self.config = cfg
        self.model = nn.Module()
        self.model.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.model.layers = nn.ModuleList([DecoderLayer(cfg, quant) for _ in range(cfg.num_layers)])
        self.model.norm = norm.RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.lm_head = None if cfg.tie_word_embeddings else nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        self.gemv_table: dict = {}

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        """input_ids [M] -> final hidden states [M, hidden] (python/tandem/models/llama_family.py:90-109)."""
        emb = self.model.embed_tokens
        hidden = emb.weight[input_ids]
        residual = None
        for layer in self.model.layers:
            hidden, residual = layer(hidden, residual)
        n = self.model.norm
        hidden, _ = norm.fused_add_rms_norm(hidden, residual, n.weight, n.eps)
        return hidden

    def compute_logits(self, hidden: torch.Tensor) -> torch.Tensor:
        """fp16 logits [M, vocab] through gemv16's table (python/tandem/models/llama_family.py:105-116,
        upcast=False)."""
        weight = self.model.embed_tokens.weight if self.lm_head is None else self.lm_head.weight
        return gemv16.linear(hidden, weight, self.gemv_table)


def prepare(model: DecoderModel, device: torch.device, device_name: Optional[str] = None) -> DecoderModel:
    """After loading: fp16 parameters on ``device``, every W4Linear repacked for this GPU, and the
    fp16 projections and logits head routed through gemv16's table."""
    model.to(device=device, dtype=torch.float16)  # W4Linear buffers keep their int32 / fp16 dtypes
    model.requires_grad_(False)  # inference only
    finalize_quantized(model, device_name)
    table = gemv16.table_for(device, model)
    gemv16.install(model, table)
    model.gemv_table = table
    return model


@torch.no_grad()
def init_random(model: DecoderModel, seed: int = 0) -> DecoderModel:
    """Synthetic weights of the architecture, generated on the model's device: AutoAWQ tensors with
    uniform int4 q and z and fp16 scales U[0.001, 0.02] (the reference tests' recipe), fp16
    projections N(0, 0.02), embeddings N(0, 1), norm weights 1 + U(-0.1, 0.1)."""
    dev = next(model.parameters()).device
    g = torch.Generator(device=dev).manual_seed(seed)
    for mod in model.modules():
        if getattr(mod, "awq_layout", False):
            for t in (mod.qweight, mod.qzeros):
                t.copy_(torch.randint(-2**31, 2**31 - 1, t.shape, device=dev, dtype=torch.int32, generator=g))
            mod.scales.copy_((torch.rand(mod.scales.shape, device=dev, generator=g) * 0.019 + 0.001).half())
    for name, p in model.named_parameters():
        if name.endswith("embed_tokens.weight"):
            p.copy_(torch.randn(p.shape, device=dev, generator=g))
        elif "norm" in name:
            p.copy_(1.0 + (torch.rand(p.shape, device=dev, generator=g) - 0.5) * 0.2)
        else:
            p.copy_(torch.randn(p.shape, device=dev, generator=g) * 0.02)
    return model
