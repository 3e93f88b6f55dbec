"""Parity helpers for the tests: the bar itself lives in oracle/parity.py
(shared with bench.py's CPU leg); printing and recording are here."""
from __future__ import annotations

import numpy as np

from oracle.parity import (MAX_ABS, MAX_REL, REL_FLOOR, argmax_rows, clause, meets_bar,  # noqa: F401
                           metrics, projection_ids)


def fmt(m: dict) -> str:
    return "  ".join(f"{k}={v:.2e}" for k, v in m.items())


def record(case: str, m: dict, **extra) -> None:
    """Print a case's parity numbers and, when FLK_PARITY_LOG names a file,
    append them to it as one JSON line (the per-configuration parity table
    is built from that file)."""
    import json
    import os
    row = {"case": case, "clause": clause(m), **{k: float(v) for k, v in m.items()}, **extra}
    print(json.dumps(row), flush=True)
    path = os.environ.get("FLK_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(row) + "\n")


def top2_margin(x: np.ndarray, rows: int) -> float:
    x = np.sort(np.asarray(x, np.float32).reshape(rows, -1), axis=1)
    return float(np.min(x[:, -1] - x[:, -2]))
