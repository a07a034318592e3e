"""Copy the reference's own data files used as golden fixtures (data only, no source).

    python tests/golden/make_fixtures.py [/root/reference]

* `dispatch_sm_90__h100-nvl-93gb_sm_90.json`: a frozen dispatch table the reference wrote
  on an H100 NVL (`results/` of the reference); it pins the table schema, the shape
  signature format and the lookup tiers against the reference's own data.
Run in the build container (the GPU box has no reference checkout); the copies are
committed.
"""
import json
import os
import shutil
import sys

FILES = ["results/dispatch_sm_90__h100-nvl-93gb_sm_90.json"]


def main() -> int:
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    here = os.path.dirname(os.path.abspath(__file__))
    for rel in FILES:
        src = os.path.join(ref, rel)
        dst = os.path.join(here, os.path.basename(rel))
        with open(src, encoding="utf-8") as f:
            json.load(f)                       # data only: must parse as JSON
        shutil.copyfile(src, dst)
        print(f"{src} -> {dst}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
