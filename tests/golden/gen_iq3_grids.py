"""Write tests/golden/iq3_grids.npz: the IQ3_XXS (256) and IQ3_S (512) grid
entries as the reference's table source states them, read as numbers from
src/iq_tables.zig (`iq3xxs_grid`, :322-355; `iq3s_grid`, :360-425).  Run in
the build container only (the reference is not on the GPU box):

    python tests/golden/gen_iq3_grids.py

The values are the data format's codebooks (ggml's grids); the fixture lets a
CPU test compare them with the oracle's grids, which come from the product's
own encoding (qwen35_amd/csrc/iq_grids.h), entry for entry.
"""
import re
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
SRC = Path("/root/reference/src/iq_tables.zig")
OUT = ROOT / "tests" / "golden" / "iq3_grids.npz"


def table(text: str, name: str, n: int) -> np.ndarray:
    """The u32 literals between `const <name>: [n]u32 ... = .{` and the closing `};`."""
    m = re.search(rf"const {name}: \[{n}\]u32[^=]*=\s*\.\{{(.*?)\}};", text, re.S)
    if m is None:
        raise SystemExit(f"{name}: declaration not found in {SRC}")
    vals = [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", m.group(1))]
    if len(vals) != n:
        raise SystemExit(f"{name}: {len(vals)} entries, expected {n}")
    return np.array(vals, np.uint32)


def main() -> None:
    text = SRC.read_text()
    np.savez(OUT, iq3xxs_grid=table(text, "iq3xxs_grid", 256), iq3s_grid=table(text, "iq3s_grid", 512))
    print(f"wrote {OUT}")


if __name__ == "__main__":
    sys.exit(main())
