"""Which kernel each dispatch site ran.

Mirrors the reference's census (``src/deepfold3/model/kernel_census.py:45-135``):
each dispatch site calls :func:`record` with the path it took, refusals are
recorded as ``refused:<reason>``, and :func:`snapshot` returns the tally.
Counts are per process and deliberately unsynchronised (a plain dict update),
like the reference's.
"""

from __future__ import annotations

import logging
from collections import defaultdict

__all__ = ["inactive", "record", "requested", "shadowed", "snapshot", "reset_counts", "reset", "format_census"]

logger = logging.getLogger(__name__)

_counts: defaultdict[str, defaultdict[str, int]] = defaultdict(lambda: defaultdict(int))
_requested: dict[str, str] = {}
_inactive: dict[str, str] = {}


def record(site: str, path: str) -> None:
    """Note that ``site`` dispatched to ``path`` once."""
    _counts[site][path] += 1


def requested(site: str, lever: str) -> None:
    """Note at construction that ``lever`` is enabled for ``site``."""
    _requested[f"{site}:{lever}"] = site


def inactive(lever: str | None = None, reason: str = "") -> dict[str, str]:
    """Note a lever gated off at construction; return all such levers."""
    if lever is not None and lever not in _inactive:
        _inactive[lever] = reason
        logger.warning("NOT ACTIVE: %s: %s", lever, reason)
    return dict(_inactive)


def snapshot() -> dict[str, dict[str, int]]:
    """The tally so far, ``{site: {path: count}}``."""
    return {site: dict(paths) for site, paths in sorted(_counts.items())}


def shadowed() -> list[str]:
    """Levers enabled at construction whose site dispatched, but never to them."""
    out = []
    for key, site in sorted(_requested.items()):
        lever = key.split(":", 1)[1]
        paths = _counts.get(site)
        if paths and lever not in paths:
            out.append(key)
    return out


def reset_counts() -> None:
    """Clear the tally, keep the requested levers."""
    _counts.clear()


def reset() -> None:
    """Clear everything (tests)."""
    _counts.clear()
    _requested.clear()
    _inactive.clear()


def format_census() -> str:
    """One line per site, plus shadowed and inactive levers."""
    lines = [f"{site}: " + ", ".join(f"{p}={n}" for p, n in sorted(paths.items())) for site, paths in snapshot().items()]
    for key in shadowed():
        lines.append(f"SHADOWED {key}")
    for lever, reason in _inactive.items():
        lines.append(f"NOT ACTIVE {lever} - {reason}")
    return "\n".join(lines) if lines else "(no kernel dispatch recorded)"
