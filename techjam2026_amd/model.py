"""The reference layer's configuration record and module tree.

`UserOptimizedTransformer` must subclass the organizer's `BaselineTransformer`
so that `copy_model_weights(..., strict=True)` keeps working
(`torch_transformer_benchmark.py:175-213`, `submission.py:40-46`). When the
organizer's script is importable its classes are used directly; otherwise this
module supplies classes with the same constructor arguments, module names and
parameter names, so a state dict moves between the two unchanged.

The `forward` methods here follow the reference's operation order
(`torch_transformer_benchmark.py:85-172`). They are not the fast path: they are
the reference answer the drop-in falls back to when the native path raises,
which is the behaviour of `submission.py:80-106`.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

try:  # the organizer's own classes, when the drop-in runs inside its script
    from torch_transformer_benchmark import (  # type: ignore
        BaselineTransformer, TransformerConfig)
    ORGANIZER_CLASSES = True
except Exception:  # pragma: no cover - the normal case in this repository
    ORGANIZER_CLASSES = False

    @dataclass(frozen=True)
    class TransformerConfig:
        """`torch_transformer_benchmark.py:29-56`: seven fields and validation."""
        batch_size: int
        seq_len: int
        d_model: int
        num_heads: int
        ffn_dim: int
        num_layers: int
        causal: bool

        def validate(self) -> None:
            for name in ("batch_size", "seq_len", "d_model", "num_heads",
                         "ffn_dim", "num_layers"):
                if getattr(self, name) <= 0:
                    raise ValueError(f"{name} must be positive")
            if self.d_model % self.num_heads != 0:
                raise ValueError(
                    f"d_model ({self.d_model}) must be divisible by "
                    f"num_heads ({self.num_heads})")

    class BaselineSelfAttention(nn.Module):
        """`torch_transformer_benchmark.py:59-122`."""

        def __init__(self, d_model: int, num_heads: int) -> None:
            super().__init__()
            if d_model % num_heads != 0:
                raise ValueError("d_model must be divisible by num_heads")
            self.d_model = d_model
            self.num_heads = num_heads
            self.head_dim = d_model // num_heads
            self.scale = self.head_dim ** -0.5
            self.q_proj = nn.Linear(d_model, d_model, bias=True)
            self.k_proj = nn.Linear(d_model, d_model, bias=True)
            self.v_proj = nn.Linear(d_model, d_model, bias=True)
            self.out_proj = nn.Linear(d_model, d_model, bias=True)

        def _heads(self, t: torch.Tensor) -> torch.Tensor:
            B, S, _ = t.shape
            return t.view(B, S, self.num_heads, self.head_dim).transpose(1, 2).contiguous()

        def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None,
                    causal: bool = False) -> torch.Tensor:
            B, S, _ = x.shape
            q = self._heads(self.q_proj(x))
            k = self._heads(self.k_proj(x))
            v = self._heads(self.v_proj(x))
            kt = k.transpose(-2, -1)
            if kt.dtype == torch.bfloat16:
                # bf16 batched products with a transposed right operand have faulted
                # MI355X GPUs; the contiguous copy leaves the product's arithmetic alone
                kt = kt.contiguous()
            scores = torch.matmul(q, kt) * self.scale
            if causal:
                upper = torch.ones((S, S), device=x.device, dtype=torch.bool).triu(1)
                scores = scores.masked_fill(upper, float("-inf"))
            if valid_token_mask is not None:
                scores = scores.masked_fill(~valid_token_mask[:, None, None, :], float("-inf"))
            probs = torch.softmax(scores.float(), dim=-1).to(dtype=x.dtype)
            ctx = torch.matmul(probs, v).transpose(1, 2).contiguous().view(B, S, self.d_model)
            out = self.out_proj(ctx)
            if valid_token_mask is not None:
                out = out.masked_fill(~valid_token_mask[..., None], 0)
            return out

    class BaselineTransformerBlock(nn.Module):
        """`torch_transformer_benchmark.py:125-145` (pre-LN, exact-erf GELU)."""

        def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
            super().__init__()
            self.norm1 = nn.LayerNorm(d_model)
            self.attention = BaselineSelfAttention(d_model, num_heads)
            self.norm2 = nn.LayerNorm(d_model)
            self.ffn_in = nn.Linear(d_model, ffn_dim)
            self.ffn_out = nn.Linear(ffn_dim, d_model)

        def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor],
                    causal: bool) -> torch.Tensor:
            x = x + self.attention(self.norm1(x), valid_token_mask, causal)
            x = x + self.ffn_out(F.gelu(self.ffn_in(self.norm2(x)), approximate="none"))
            if valid_token_mask is not None:
                x = x.masked_fill(~valid_token_mask[..., None], 0)
            return x

    class BaselineTransformer(nn.Module):
        """`torch_transformer_benchmark.py:148-172`."""

        def __init__(self, config: TransformerConfig) -> None:
            super().__init__()
            self.config = config
            self.layers = nn.ModuleList([
                BaselineTransformerBlock(config.d_model, config.num_heads, config.ffn_dim)
                for _ in range(config.num_layers)])
            self.final_norm = nn.LayerNorm(config.d_model)

        def forward(self, x: torch.Tensor,
                    valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
            for layer in self.layers:
                x = layer(x, valid_token_mask, self.config.causal)
            x = self.final_norm(x)
            if valid_token_mask is not None:
                x = x.masked_fill(~valid_token_mask[..., None], 0)
            return x


__all__ = ["TransformerConfig", "BaselineTransformer", "ORGANIZER_CLASSES"]
