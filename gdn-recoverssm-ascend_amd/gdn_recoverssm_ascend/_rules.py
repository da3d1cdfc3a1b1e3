"""Declarative argument checks for the host API and the torch operators.

A rule is a pair (message, predicate). ``enforce`` evaluates the predicates of
a rule table in order and raises ``ValueError("GDN RecoverSSM: <message>")``
for the first one that fails, before anything is launched. Tables are ordered
so that a predicate may rely on what the rules above it established (a rank
before a shape, a shape before a stride).
"""

from __future__ import annotations

from collections.abc import Callable, Iterable

PREFIX = "GDN RecoverSSM: "

Rule = tuple[str, Callable[..., bool]]


def fail(message: str) -> None:
    raise ValueError(PREFIX + message)


def require(condition: bool, message: str) -> None:
    """One rule, evaluated on the spot."""
    if not condition:
        fail(message)


def enforce(rules: Iterable[Rule], *subject, where: str = "") -> None:
    """Raise for the first rule whose predicate is false on ``subject``."""
    for message, predicate in rules:
        if not predicate(*subject):
            fail(f"{where}: {message}" if where else message)
