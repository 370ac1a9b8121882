"""Writes diag_signs_seed42.json: PolarQuant's Rademacher diagonal for the engine's seed (42) at the
two dims on the path (d = 128 KV blocks, d = 64 index keys), as the reference builds it
(aether_2b/turbo_quant.py:111-121): torch.Generator().manual_seed(seed * 10007 + d), r = torch.rand(d),
+1 where r > 0.5 else -1.  Only torch's CPU generator is run; the reference itself is not imported.

    python tests/golden/make_diag_signs.py
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

SEED = 42


def signs(seed: int, d: int) -> str:
    g = torch.Generator()
    g.manual_seed(seed * 10007 + d)
    r = torch.rand(d, generator=g)
    return "".join("+" if v > 0.5 else "-" for v in r.tolist())


def main() -> None:
    out = {"seed": SEED, "generator_seed": {str(d): SEED * 10007 + d for d in (64, 128)},
           "signs": {str(d): signs(SEED, d) for d in (64, 128)}, "torch": torch.__version__}
    path = Path(__file__).with_name("diag_signs_seed42.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
