"""Argument contracts of the public operators, as data.

Every public entry point of this package checks its arguments before any
launch, raising ``TypeError`` for a wrong type or dtype and ``ValueError`` for
a wrong shape, layout, device or value. The exception types, messages and the
order in which the checks run are part of the reference's API (reference
callers and tests match them; e.g. ``tests/tmix/wkv7/test.py:644-720``), so
they are kept exactly. How the checks are written is this package's own: each
entry point owns a table of :class:`Rule` / :class:`Each` steps and calls
:func:`enforce` on its arguments. A rule is a predicate over the argument
namespace plus the error it raises; :class:`Each` applies a list of rules to
several arguments in turn (argument-major order, which is the order the
reference checks its per-tensor lists in).

Predicates receive ``(value, ns)`` where ``ns`` maps argument names to
values, so cross-argument conditions ("shares r's device") are one-liners.
A predicate returns True when the argument is acceptable.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Callable, Iterable, Mapping, Sequence

import torch

Pred = Callable[[Any, Mapping[str, Any]], bool]


@dataclass(frozen=True)
class Rule:
    """Check argument ``arg`` (``None``: the rule looks at ``ns`` only)."""

    arg: str | None
    ok: Pred
    error: type
    message: str

    def run(self, ns: Mapping[str, Any], name: str | None = None) -> None:
        target = self.arg if name is None else name
        value = ns.get(target) if target is not None else None
        if not self.ok(value, ns):
            raise self.error(self.message.format(name=target))


@dataclass(frozen=True)
class Each:
    """Apply ``rules`` to each of ``args``, all rules for one argument first."""

    args: tuple[str, ...]
    rules: tuple[Rule, ...]

    def run(self, ns: Mapping[str, Any]) -> None:
        for name in self.args:
            for rule in self.rules:
                rule.run(ns, name)


Step = "Rule | Each"


def enforce(steps: Iterable, ns: Mapping[str, Any]) -> None:
    """Run the steps of a contract table over the argument namespace."""
    for step in steps:
        step.run(ns)


# ---------------------------------------------------------------- predicates
def tensor(x, ns) -> bool:
    return isinstance(x, torch.Tensor)


def contiguous(x, ns) -> bool:
    return x.is_contiguous()


def cuda_contiguous(x, ns) -> bool:
    return x.is_cuda and x.is_contiguous()


def dtype_is(*dtypes: torch.dtype) -> Pred:
    return lambda x, ns: x.dtype in dtypes


def ndim_is(n: int) -> Pred:
    return lambda x, ns: x.ndim == n


def same_device_as(other: str) -> Pred:
    return lambda x, ns: x.device == ns[other].device


def same_shape_as(other: str) -> Pred:
    return lambda x, ns: x.shape == ns[other].shape


def positive_int(x, ns) -> bool:
    return isinstance(x, int) and not isinstance(x, bool) and x > 0


def plain_int(x, ns) -> bool:
    return isinstance(x, int) and not isinstance(x, bool)


def finite_number(x, ns) -> bool:
    return isinstance(x, (int, float)) and math.isfinite(float(x))


def finite(x, ns) -> bool:
    return math.isfinite(float(x))


def one_of(values: Sequence) -> Pred:
    return lambda x, ns: x in values


def packed_rows(x, ns) -> bool:
    """[total_tokens, C] with both dimensions non-empty."""
    return x.ndim == 2 and x.shape[0] > 0 and x.shape[1] > 0


# ------------------------------------------------------------- rule builders
def is_tensor(arg: str | None = None) -> Rule:
    return Rule(arg, tensor, TypeError, "{name} must be a torch.Tensor")


def check(arg: str | None, ok: Pred, error: type, message: str) -> Rule:
    return Rule(arg, ok, error, message)


def when(cond: Callable[[Mapping[str, Any]], bool], rule: Rule) -> Rule:
    """``rule`` that only applies when ``cond(ns)`` holds."""
    return Rule(rule.arg, lambda x, ns: (not cond(ns)) or rule.ok(x, ns), rule.error,
                rule.message)


# Argument lists shared by the WKV7 entries.
PACKED_TOKENS = ("r", "decay_logits", "k", "v", "a", "b")

# Metadata pair of the recurrent family (reference ``tmix/wkv7/__init__.py:154-163``).
METADATA = (
    is_tensor("cu_seqlens"),
    check("cu_seqlens", ndim_is(1), ValueError, "cu_seqlens must be one-dimensional"),
    is_tensor("state_indices"),
)


def native():
    """The loaded native facade, or RuntimeError when it is not built."""
    import flashrwkv_amd

    facade = getattr(flashrwkv_amd, "_C", None)
    if facade is None:
        raise RuntimeError(
            "flashrwkv_amd native extension is not built; run "
            "`python -m flashrwkv_amd._build` before using the WKV7 operators"
        )
    return facade
