"""Competition entry point: the drop-in `UserOptimizedTransformer`.

Interface and behaviour fixed by the organizer's harness and the reference's
`submission.py:40-106`:

* subclasses `BaselineTransformer`, so the organizer's `copy_model_weights(strict=True)`
  keeps working (parameter names and module tree unchanged, only `forward` replaced);
* on the first forward, probes the device, looks the shape up in the gfx950 dispatch
  table (`DispatchTable.load_for(spec).lookup(arch, dtype, config, lds_kb)`), builds a
  `FusedTransformer` with the chosen plan and copies the weights into it;
* any exception while choosing or running the plan is reported once on stdout and the
  module then serves every later call with the reference forward: an error in the fast
  path costs speed, never a wrong or missing answer.

`KERNELFORGE_PLAN` forces a ladder plan and `KERNELFORGE_VERBOSE` prints the choice (the
reference's variables). `KF950_STRICT=1` re-raises instead of falling back (used by tests
that must prove the native path ran).
"""
from __future__ import annotations

import os
from typing import Optional, Tuple

import torch

from .dispatch import DispatchTable
from .hw import probe
from .model import BaselineTransformer, TransformerConfig, reference_forward
from .optimized import LADDER, FusedTransformer, Plan

_FORCED = os.environ.get("KERNELFORGE_PLAN")
_VERBOSE = os.environ.get("KERNELFORGE_VERBOSE", "") not in ("", "0")


def _strict() -> bool:
    return os.environ.get("KF950_STRICT", "") not in ("", "0")


def _choose_plan(dtype: torch.dtype, config: TransformerConfig) -> Tuple[Plan, str, str]:
    """(plan, where it came from, device arch) for this module's shape and I/O dtype."""
    spec = probe(measure=False)
    if _FORCED:
        return LADDER[_FORCED], f"env:{_FORCED}", spec.arch
    table = DispatchTable.load_for(spec)
    plan, source = table.lookup(spec.arch, dtype, config, spec.shared_mem_per_block_kb)
    return plan, source, spec.arch


class UserOptimizedTransformer(BaselineTransformer):
    def __init__(self, config: TransformerConfig) -> None:
        super().__init__(config)
        self._impl: Optional[FusedTransformer] = None
        self._plan: Optional[Plan] = None
        self._source = "uninitialized"
        self._failed = False

    def _give_up(self, when: str, err: Exception) -> None:
        """Switch this module to the reference forward for good, saying why once."""
        self._failed, self._impl = True, None
        print(f"[kernelforge] native gfx950 path unavailable ({when}: "
              f"{type(err).__name__}: {err}); this module now runs the PyTorch "
              f"reference forward for every call")

    def _select(self, dtype: torch.dtype) -> None:
        if self._impl is not None or self._failed:
            return
        try:
            plan, source, arch = _choose_plan(dtype, self.config)
            native = FusedTransformer(self.config, plan)
            native.load_state_dict(self.state_dict(), strict=True)
            device = next(self.parameters()).device
            self._impl = native.to(device, dtype).eval()
            self._plan, self._source = plan, source
            if _VERBOSE:
                print(f"[kernelforge] {arch} {dtype}: plan {plan.name} from the {source} "
                      f"table entry -- {plan.describe()}")
        except Exception as err:
            if _strict():
                raise
            self._give_up("plan selection", err)

    def forward(self, x: torch.Tensor,
                valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        self._select(x.dtype)
        native = self._impl
        if native is not None:
            try:
                return native(x, valid_token_mask)
            except Exception as err:
                if _strict():
                    raise
                self._give_up("forward", err)
        # the reference forward over this module's own parameters (restated op for op,
        # with the bf16 transposed-operand product avoided)
        return reference_forward(self, x, valid_token_mask)
