"""A per-process ledger of which kernel path each dispatch site took.

Public interface as in the reference's census (``src/deepfold3/model/kernel_census.py``;
callers such as its ``scripts/inference.py:957-959`` write ``snapshot()``,
``shadowed()`` and ``inactive()`` into run manifests):

- ``record(site, path)``: one dispatch of ``site`` through ``path``; refusals use the
  path ``"refused:<reason>"``.
- ``requested(site, lever)``: a lever was enabled for ``site`` at construction.
- ``shadowed()``: ``"site:lever"`` for every requested lever whose site has dispatched,
  but never through that lever. A path ``"<lever>_<variant>"`` (``"hip_tri_attn_row"``
  for the lever ``"hip"``) counts as the lever's.
- ``inactive(lever, reason)``: a lever gated off at construction (logged once); with no
  argument, the levers gated off so far.
- ``snapshot()`` ``{site: {path: count}}``, ``format_census()`` a readable summary,
  ``reset_counts()`` / ``reset()``, ``warn_once(key)``.

Here the ledger is one object holding a ``Counter`` over ``(site, path)`` pairs, updated
under a lock, so concurrent dispatch from several threads (the trunk's second stream is
driven from the same thread, but callers may use more) keeps exact counts.
"""

from __future__ import annotations

import logging
import threading
from collections import Counter

__all__ = [
    "record",
    "requested",
    "inactive",
    "snapshot",
    "shadowed",
    "warn_once",
    "reset_counts",
    "reset",
    "format_census",
]

_log = logging.getLogger(__name__)


class _Ledger:
    def __init__(self) -> None:
        self.lock = threading.Lock()
        self.hits: Counter[tuple[str, str]] = Counter()
        self.levers: set[tuple[str, str]] = set()  # (site, lever) enabled at construction
        self.gated: dict[str, str] = {}  # lever -> reason, in the order first seen
        self.warned: set[str] = set()

    def paths_of(self, site: str) -> set[str]:
        return {p for (s, p) in self.hits if s == site}


_LEDGER = _Ledger()


def record(site: str, path: str) -> None:
    """Count one dispatch of ``site`` through ``path``."""
    with _LEDGER.lock:
        _LEDGER.hits[(site, path)] += 1


def requested(site: str, lever: str) -> None:
    """Remember that ``lever`` is enabled for ``site`` (called at construction)."""
    with _LEDGER.lock:
        _LEDGER.levers.add((site, lever))


def inactive(lever: str | None = None, reason: str = "") -> dict[str, str]:
    """Register ``lever`` as gated off for ``reason`` (first registration wins and is
    logged); return every gated lever with its reason."""
    with _LEDGER.lock:
        new = lever is not None and lever not in _LEDGER.gated
        if new:
            _LEDGER.gated[lever] = reason
        gated = dict(_LEDGER.gated)
    if new:
        _log.warning("kernel lever %s is gated off: %s", lever, reason)
    return gated


def snapshot() -> dict[str, dict[str, int]]:
    """``{site: {path: count}}``, sites and paths in sorted order."""
    with _LEDGER.lock:
        items = sorted(_LEDGER.hits.items())
    out: dict[str, dict[str, int]] = {}
    for (site, path), n in items:
        out.setdefault(site, {})[path] = n
    return out


def shadowed() -> list[str]:
    """Requested levers whose site dispatched but never through them, as ``site:lever``."""
    with _LEDGER.lock:
        levers = sorted(_LEDGER.levers)
        taken = {site: _LEDGER.paths_of(site) for site, _ in levers}

    def used(lever: str, paths: set[str]) -> bool:
        return any(p == lever or p.startswith(lever + "_") for p in paths)

    return [f"{site}:{lever}" for site, lever in levers if taken[site] and not used(lever, taken[site])]


def warn_once(key: str) -> bool:
    """True the first time ``key`` is seen in this process, False afterwards."""
    with _LEDGER.lock:
        if key in _LEDGER.warned:
            return False
        _LEDGER.warned.add(key)
        return True


def reset_counts() -> None:
    """Forget the dispatch counts; keep requested and gated levers."""
    with _LEDGER.lock:
        _LEDGER.hits.clear()


def reset() -> None:
    """Forget everything (for tests)."""
    with _LEDGER.lock:
        _LEDGER.hits.clear()
        _LEDGER.levers.clear()
        _LEDGER.gated.clear()
        _LEDGER.warned.clear()


def format_census() -> str:
    """A summary: one ``site  path xN`` line per path, then shadowed and gated levers."""
    snap = snapshot()
    rows = [f"{site}  {path} x{n}" for site, paths in snap.items() for path, n in paths.items()]
    rows += [f"shadowed lever: {key}" for key in shadowed()]
    rows += [f"gated lever: {lever} ({why})" for lever, why in inactive().items()]
    return "\n".join(rows) if rows else "no kernel dispatch recorded"
