"""Golden fixtures from the reference's own data (tests/golden/, copied there by
`tests/golden/make_fixtures.py`): the dispatch table the reference froze on an H100 NVL
(`results/dispatch_sm_90__h100-nvl-93gb_sm_90.json`). It pins, against the reference's
data rather than a restatement, the table entry schema (`kernelforge/dispatch.py:92-109`),
the shape-signature format (`:40-44`) and the lookup tiers (`:254-288`).
"""
from __future__ import annotations

import json
import os
import re

import torch

from techjam2026_amd.dispatch import DispatchTable, Entry, default_plan, shape_signature
from techjam2026_amd.model import TransformerConfig

GOLDEN = os.path.join(os.path.dirname(__file__), "golden",
                      "dispatch_sm_90__h100-nvl-93gb_sm_90.json")


def _blob() -> dict:
    with open(GOLDEN, encoding="utf-8") as f:
        return json.load(f)


def _cfg(sig: str) -> TransformerConfig:
    m = re.fullmatch(r"B(\d+)-S(\d+)-d(\d+)-H(\d+)-F(\d+)-L(\d+)(-causal)?", sig)
    assert m, sig
    b, s, d, h, f, layers, causal = m.groups()
    return TransformerConfig(int(b), int(s), int(d), int(h), int(f), int(layers), causal is not None)


def test_reference_table_entries_load_and_write_back_field_for_field():
    blob = _blob()
    entries = [Entry.from_json(e) for e in blob["entries"]]
    assert blob["arch"] == "sm_90" and len(entries) == 13
    for raw, e in zip(blob["entries"], entries):
        assert e.plan.name == raw["plan"]["name"]
        assert [list(o) for o in e.plan.overrides] == raw["plan"]["overrides"]
        assert e.plan.torch_compile == raw["plan"]["torch_compile"]
        back = e.to_json()
        for k in ("signature", "dtype", "arch", "regime", "utilization", "speedup",
                  "speedup_vs_compile", "case"):
            assert back[k] == raw[k], k
        for k, v in raw["plan"].items():
            assert back["plan"][k] == v, (raw["signature"], k)


def test_reference_signatures_are_our_shape_signatures():
    for raw in _blob()["entries"]:
        assert shape_signature(_cfg(raw["signature"])) == raw["signature"]


def test_lookup_tiers_on_the_reference_table():
    blob = _blob()
    table = DispatchTable([Entry.from_json(e) for e in blob["entries"]])
    for raw in blob["entries"]:
        plan, src = table.lookup("sm_90", torch.float32, _cfg(raw["signature"]), smem_kb=160.0)
        assert src == "exact" and plan.name == raw["plan"]["name"]
        assert plan.smem_kb == 160.0            # the card's LDS budget replaces the stored one
    # same arch and dtype, unseen shape: the conservative default
    plan, src = table.lookup("sm_90", torch.float32, TransformerConfig(3, 100, 128, 4, 128, 4, True))
    assert src == "nearest"
    assert plan == default_plan(torch.float32, conservative=True, arch="sm_90")
    # another architecture, or a dtype the table has no entry for: the default rule
    assert table.lookup("gfx950", torch.float32, _cfg(blob["entries"][0]["signature"]))[1] == "default"
    assert table.lookup("sm_90", torch.float16, _cfg(blob["entries"][0]["signature"]))[1] == "default"
