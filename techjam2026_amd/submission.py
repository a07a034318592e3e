"""Competition entry point: the drop-in `UserOptimizedTransformer`.

Behaviour of the reference's `submission.py:40-106`:

* subclasses `BaselineTransformer`, so the organizer's `copy_model_weights(strict=True)`
  keeps working (parameter names and module tree unchanged, only `forward` replaced);
* on the first forward, probes the device, looks the shape up in the gfx950 dispatch
  table (`DispatchTable.load_for(spec).lookup(arch, dtype, config, lds_kb)`), builds a
  `FusedTransformer` with the chosen plan and copies the weights into it;
* any exception while choosing or running the plan prints an announcement and falls
  back, permanently, to the reference forward -- the right answer, not a traceback.

`KERNELFORGE_PLAN` forces a ladder plan and `KERNELFORGE_VERBOSE` prints the choice, as
in the reference. `KF950_STRICT=1` re-raises instead of falling back (used by tests
that must prove the native path ran).
"""
from __future__ import annotations

import os
from typing import Optional

import torch

from .dispatch import DispatchTable
from .hw import probe
from .model import BaselineTransformer, TransformerConfig
from .optimized import LADDER, FusedTransformer, Plan

_FORCED = os.environ.get("KERNELFORGE_PLAN")
_VERBOSE = os.environ.get("KERNELFORGE_VERBOSE", "") not in ("", "0")


def _strict() -> bool:
    return os.environ.get("KF950_STRICT", "") not in ("", "0")


class UserOptimizedTransformer(BaselineTransformer):
    def __init__(self, config: TransformerConfig) -> None:
        super().__init__(config)
        self._impl: Optional[FusedTransformer] = None
        self._plan: Optional[Plan] = None
        self._source = "uninitialized"
        self._failed = False

    def _select(self, dtype: torch.dtype) -> None:
        if self._impl is not None or self._failed:
            return
        try:
            spec = probe(measure=False)
            lds = spec.shared_mem_per_block_kb
            if _FORCED:
                plan, source = LADDER[_FORCED], f"env:{_FORCED}"
            else:
                table = DispatchTable.load_for(spec)
                plan, source = table.lookup(spec.arch, dtype, self.config, lds)
            impl = FusedTransformer(self.config, plan)
            impl.load_state_dict(self.state_dict(), strict=True)
            impl = impl.to(next(self.parameters()).device, dtype).eval()
            self._impl, self._plan, self._source = impl, plan, source
            if _VERBOSE:
                print(f"[kernelforge] {spec.arch} {dtype} -> {plan.name} ({source}): "
                      f"{plan.describe()}")
        except Exception as e:
            if _strict():
                raise
            self._failed = True
            print(f"[kernelforge] falling back to baseline: {type(e).__name__}: {e}")

    def forward(self, x: torch.Tensor,
                valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        self._select(x.dtype)
        if self._impl is None:
            return super().forward(x, valid_token_mask)
        try:
            return self._impl(x, valid_token_mask)
        except Exception as e:
            if _strict():
                raise
            self._failed, self._impl = True, None
            print(f"[kernelforge] the fused path raised {type(e).__name__}: {e}"
                  f"\n[kernelforge] falling back to the reference implementation "
                  f"for the rest of this run; results stay correct, speed does not.")
            return super().forward(x, valid_token_mask)
