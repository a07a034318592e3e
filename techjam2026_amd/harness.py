"""Synthetic inputs and weights, as the organizer's harness draws them.

* `generate_random_case` follows `torch_transformer_benchmark.py:234-272`:
  x ~ N(0,1) * input_scale; with padding, per-sequence valid lengths
  ~ randint[max(1, round(S * (1 - p))), S]; mask = position < length; padded
  rows of x zeroed. The draw always happens on a CPU generator and the result
  is then moved to `device`, so a CPU baseline and a GPU run see the same
  numbers (the organizer draws on the target device, whose stream differs
  between CPU and GPU).
* `init_weights_` applies `xavier_uniform_` to every Linear weight from a seed
  (BASELINE configs say Xavier); biases keep nn.Linear's default
  (seeded) init, LayerNorm weight/bias are 1/0, or random when
  `random_norms=True` so that LN(0) = beta is visible in tests.
* `copy_model_weights` is `torch_transformer_benchmark.py:203-213`.
"""
from __future__ import annotations

import copy
from typing import Optional, Tuple

import torch
import torch.nn as nn


def generate_random_case(config, device, dtype: torch.dtype, seed: int,
                         padding_ratio: float, input_scale: float = 1.0,
                         ) -> Tuple[torch.Tensor, torch.Tensor]:
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    B, S, d = config.batch_size, config.seq_len, config.d_model
    x = torch.randn(B, S, d, generator=gen, dtype=torch.float32)
    x = x * input_scale
    if padding_ratio <= 0:
        mask = torch.ones(B, S, dtype=torch.bool)
    else:
        min_valid = max(1, int(round(S * (1.0 - padding_ratio))))
        lengths = torch.randint(low=min_valid, high=S + 1, size=(B,), generator=gen)
        mask = torch.arange(S)[None, :] < lengths[:, None]
        x = x.masked_fill(~mask[..., None], 0)
    return x.to(device=device, dtype=dtype), mask.to(device)


def init_weights_(model: nn.Module, seed: int, random_norms: bool = False) -> nn.Module:
    """Seeded re-initialisation in place; deterministic for a given seed."""
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    with torch.no_grad():
        for mod in model.modules():
            if isinstance(mod, nn.Linear):
                fan_in = mod.weight.shape[1]
                w = torch.empty(mod.weight.shape, dtype=torch.float32)
                nn.init.xavier_uniform_(w, generator=gen)
                bound = 1.0 / fan_in ** 0.5       # nn.Linear's default bias bound
                b = (torch.rand(mod.bias.shape, generator=gen) * 2 - 1) * bound
                mod.weight.copy_(w)
                mod.bias.copy_(b)
            elif isinstance(mod, nn.LayerNorm):
                if random_norms:
                    mod.weight.copy_(1.0 + 0.2 * torch.randn(mod.weight.shape, generator=gen))
                    mod.bias.copy_(0.2 * torch.randn(mod.bias.shape, generator=gen))
                else:
                    mod.weight.fill_(1.0)
                    mod.bias.zero_()
    return model


def copy_model_weights(baseline: nn.Module, optimized: nn.Module,
                       strict: bool = True) -> None:
    state = copy.deepcopy(baseline.state_dict())
    optimized.load_state_dict(state, strict=strict)


def padding_ratio_for(config_index: int) -> float:
    """Padding ratio of BASELINE configs C1..C5 (index 0..4).

    The valid-length ranges they state map to the generator's
    min_valid = round(S * (1 - p)): C1 [S/2,S] -> 0.5, C2 [64,512] -> 0.875,
    C3 [128,1024] -> 0.875, C4 [S/4,S] -> 0.75, C5 [S/2,S] -> 0.5.
    """
    return (0.5, 0.875, 0.875, 0.75, 0.5)[config_index]


def lengths_of(mask: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if mask is None else mask.long().sum(dim=1)
