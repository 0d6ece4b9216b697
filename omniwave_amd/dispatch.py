"""Backend selection with automatic fallback (omniweave/ops/dispatch.py:13-49).

The accelerated backend is ``"hip"`` (the reference's is ``"triton"``); otherwise the
contract is the reference's: unknown names raise ValueError, a forced accelerated backend
that is unsupported raises RuntimeError(reason), and ``"auto"`` logs the reason and falls
back to ``"reference"``.
"""

from __future__ import annotations

import logging
from collections.abc import Callable

from torch import Tensor

logger = logging.getLogger(__name__)

BACKENDS = frozenset({"reference", "compile", "hip", "auto"})


def select_backend(
    x: Tensor,
    requested: str,
    support_check: Callable[[Tensor], tuple[bool, str | None]],
) -> tuple[str, str | None]:
    """Return ``(backend, fallback_reason)`` for ``requested``.

    ``support_check(x)`` returns ``(is_supported, reason_if_not)`` for the hip backend.
    """
    if requested not in BACKENDS:
        raise ValueError(f"unknown backend: {requested!r}")
    if requested in {"reference", "compile"}:
        return requested, None
    supported, reason = support_check(x)
    if supported:
        return "hip", None
    if requested == "hip":
        raise RuntimeError(reason)
    logger.info("falling back to reference backend: %s", reason)
    return "reference", reason
