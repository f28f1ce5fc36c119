"""Loader for fp8_gfx942_rocm.golden: the reference's gfx942 FNUZ fp8 golden
fixture (crates/fe2o3-device/tests/fixtures/fp8_gfx942_rocm.golden, read by
crates/fe2o3-device/tests/fp8_gfx942_golden.rs), kept here as data.  Native
gfx942 conversions (ROCm 7.2.4) of:
  widen  <e4|e5> <code> <f32 bits>                    256 per format
  narrow <e4|e5> <case> <f32 bits> <code>             1046 per format
  pack   <e4|e5> <case> <lane0> .. <lane3> <u32>      7 per format
Format index: e4 -> 0 (E4M3 FNUZ), e5 -> 1 (E5M2 FNUZ)."""
from __future__ import annotations

import os

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fp8_gfx942_rocm.golden")
FORMATS = {"e4": 0, "e5": 1}


def load(path: str = PATH) -> dict:
    out = {"meta": {}, "widen": [], "narrow": [], "pack": []}
    with open(path) as f:
        for line in f:
            t = line.split()
            if not t:
                continue
            if t[0] == "meta":
                out["meta"][t[1]] = " ".join(t[2:])
            elif t[0] == "widen":
                out["widen"].append((FORMATS[t[1]], int(t[2], 16), int(t[3], 16)))
            elif t[0] == "narrow":
                out["narrow"].append((FORMATS[t[1]], t[2], int(t[3], 16), int(t[4], 16)))
            elif t[0] == "pack":
                out["pack"].append((FORMATS[t[1]], t[2], [int(x, 16) for x in t[3:7]],
                                    int(t[7], 16)))
            else:
                raise ValueError(f"unknown record {t[0]!r}")
    return out
