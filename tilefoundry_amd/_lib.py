"""Loads the native extension. There is no fallback: without the built HIP
library every op raises at import time, naming the build command."""
from __future__ import annotations

try:
    from . import _C  # noqa: F401  (the torch extension; links libtilefoundry_amd.so)
except ImportError as exc:  # pragma: no cover - exercised only on a broken install
    raise ImportError(
        "tilefoundry_amd: the native extension is not built or failed to load "
        f"({exc}). Build it with `python -m tilefoundry_amd._build`."
    ) from exc

C = _C
