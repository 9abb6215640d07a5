"""Parity metrics of the GPU tests against the fp64 oracle.

Every comparison reports three figures of the kernel result x against the
oracle's x_ref (fp64):

* normwise: ``max|x - x_ref| / max|x_ref|`` (``oracle.max_rel_error``), the
  metric the north star's tolerances (1e-5 fp32, 2e-2 bf16) are stated in;
* per row: the worst row of the last axis (the D features of one token-head,
  or one key row of a state), each row's max error divided by
  ``max(max|x_ref_row|, ROW_FLOOR * max over rows)`` (ROW_FLOOR = 1e-2). A
  row that is wrong relative to its own scale fails here even when it is
  small against the tensor's largest row (a strongly decayed state's tail,
  low-norm rows of a gradient);
* elementwise with a floor: ``max_i |x_i - x_ref_i| / max(|x_ref_i|,
  floor * max|x_ref|)``. The error of one element of a bf16 product is set by
  the magnitudes of the terms summed into it, not by its own value (sums
  cancel), so the floor each test states is the fraction of the tensor's
  largest entry below which an element is judged absolutely. This is the
  reference tests' ``allclose(x, ref, atol, rtol)`` form with ``rtol = tol``
  and ``atol = tol * floor * max|x_ref|`` (the reference states atol in
  absolute units for its own input scales).

``FRWKV_PARITY_LOG=<path>`` appends one JSON line per comparison with all
three figures (elementwise at several floors), which is how the stated
bounds were chosen.
"""

from __future__ import annotations

import json
import os

import numpy as np

ROW_FLOOR = 1e-2
LOG_FLOORS = (1e-3, 3e-3, 1e-2, 3e-2, 1e-1, 3e-1)
LOG_ROW_FLOORS = (1e-3, 1e-2, 3e-2, 1e-1)


def as_f64(x) -> np.ndarray:
    if hasattr(x, "detach"):
        x = x.detach().double().cpu().numpy()
    return np.asarray(x, dtype=np.float64)


def normwise(actual, expected) -> float:
    actual, expected = as_f64(actual), as_f64(expected)
    if expected.size == 0:
        return 0.0
    denom = float(np.max(np.abs(expected))) or 1.0
    return float(np.max(np.abs(actual - expected)) / denom)


def elementwise(actual, expected, floor: float) -> float:
    actual, expected = as_f64(actual), as_f64(expected)
    if expected.size == 0:
        return 0.0
    scale = float(np.max(np.abs(expected))) or 1.0
    denom = np.maximum(np.abs(expected), floor * scale)
    return float(np.max(np.abs(actual - expected) / denom))


def rowwise(actual, expected, floor: float = ROW_FLOOR) -> float:
    actual, expected = as_f64(actual), as_f64(expected)
    if expected.size == 0:
        return 0.0
    width = expected.shape[-1] if expected.ndim else 1
    e = expected.reshape(-1, width)
    d = np.abs(actual.reshape(-1, width) - e).max(axis=1)
    row_scale = np.abs(e).max(axis=1)
    denom = np.maximum(row_scale, floor * (float(row_scale.max()) or 1.0))
    return float(np.max(d / denom))


def _log(name: str, actual, expected, norm: float) -> None:
    path = os.environ.get("FRWKV_PARITY_LOG")
    if not path:
        return
    import inspect

    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]
    caller = inspect.stack()[2]
    record = {
        "test": test,
        "site": f"{os.path.basename(caller.filename)}:{caller.lineno}",
        "name": name,
        "norm": norm,
        "row": rowwise(actual, expected),
        "rows": {f"{f:g}": rowwise(actual, expected, f) for f in LOG_ROW_FLOORS},
        "elem": {f"{f:g}": elementwise(actual, expected, f) for f in LOG_FLOORS},
    }
    with open(path, "a") as fh:
        fh.write(json.dumps(record) + "\n")


def check(name: str, actual, expected, tol: float, *, row_tol: float | None = None,
          elem_tol: float | None = None, elem_floor: float | None = None) -> float:
    """Assert the normwise bound ``tol`` and, where given, the per-row and
    elementwise bounds; returns the normwise error."""
    actual, expected = as_f64(actual), as_f64(expected)
    assert np.isfinite(actual).all(), f"{name}: non-finite values"
    norm = normwise(actual, expected)
    _log(name, actual, expected, norm)
    msg = f"{name}: max-rel {norm:.3e}"
    assert norm <= tol, f"{msg} > {tol}"
    if row_tol is not None:
        row = rowwise(actual, expected)
        msg += f" row {row:.3e}"
        assert row <= row_tol, f"{name}: per-row {row:.3e} > {row_tol}"
    if elem_tol is not None:
        assert elem_floor is not None
        elem = elementwise(actual, expected, elem_floor)
        msg += f" elem@{elem_floor:g} {elem:.3e}"
        assert elem <= elem_tol, (f"{name}: elementwise (floor {elem_floor:g}) {elem:.3e} > "
                                  f"{elem_tol}")
    print(msg)
    return norm
