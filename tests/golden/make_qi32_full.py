"""Writes tests/golden/qi32_full.json: sha256 of the int32 outputs of the reference's own
cpu_fprop_nhwc_qi32 (/root/reference/src/cpu_ref.cpp:36-72, compiled unmodified into
oracle/_ref/libref_cpu.so by oracle/Makefile) on the full-size float-code problems of
tests.golden.cases.QI32_FULL, after checking that the oracle's C restatement gives the same
bits.  Run in the build container (the GPU box has no /root/reference):

    make -C oracle && python tests/golden/make_qi32_full.py
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from tests.golden.cases import QI32_FULL, qi32_full_inputs  # noqa: E402

OUT = Path(__file__).resolve().parent / "qi32_full.json"


def main() -> None:
    if oracle.ref() is None:
        raise SystemExit("build oracle/_ref first: make -C oracle (needs /root/reference)")
    res = {}
    for name in QI32_FULL:
        kind, x, w, conv, zp, fzp = qi32_full_inputs(name)
        y, secs = oracle.ref_conv_qi32(kind, x, w, conv, zp, fzp)
        mine = oracle.conv_qi32(x, w, conv, zp, fzp)
        if not np.array_equal(y, mine):
            raise SystemExit(f"{name}: the oracle's restatement differs from the reference")
        res[name] = {"shape": list(y.shape), "sha256": hashlib.sha256(np.ascontiguousarray(y).tobytes()).hexdigest(),
                     "ref_seconds": round(secs, 2)}
        print(name, res[name], flush=True)
    with open(OUT, "w") as f:
        json.dump(res, f, indent=1)
    print("written", OUT)


if __name__ == "__main__":
    main()
