"""Opt-in ``rosellm`` namespace over this package.

``import rosellm.roserlhf`` (and ``rosellm.roserlhf.losses``, ``.advantages``,
``.trajectory``) then resolves to ``rosellm_amd.roserlhf``, so code written
against the reference runs unchanged.  Nothing is importable as ``rosellm``
until a caller opts in, and the shim never stands in for an installed
reference:

* ``enable()`` appends the shim's directory to the end of ``sys.path``: a
  ``rosellm`` found earlier on the path (the reference) keeps winning;
* ``install(directory)`` copies the shim package into ``directory`` (for a
  scratch or virtual-environment path the caller puts on ``sys.path``);
* the shim's ``rosellm/__init__.py`` raises ImportError if another
  ``rosellm`` is importable from ``sys.path`` anyway (the shim listed first).

Only ``rosellm.roserlhf`` is provided (the hot path this package implements).
"""

from __future__ import annotations

import shutil
import sys
from pathlib import Path

SITE = Path(__file__).resolve().parent / "site"


def enable() -> str:
    """Put the shim at the end of ``sys.path`` (idempotent); returns that entry."""

    entry = str(SITE)
    if entry not in sys.path:
        sys.path.append(entry)
    return entry


def install(directory) -> Path:
    """Copy the shim package into ``directory`` (created if needed) as
    ``directory/rosellm``; returns ``directory``."""

    target = Path(directory)
    target.mkdir(parents=True, exist_ok=True)
    dest = target / "rosellm"
    if dest.exists():
        raise FileExistsError(f"{dest} exists; the shim is not copied over another package")
    shutil.copytree(SITE / "rosellm", dest,
                    ignore=shutil.ignore_patterns("__pycache__", "*.pyc"))
    return target
