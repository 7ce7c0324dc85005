"""``rosellm`` namespace of rosellm_amd's opt-in shim: only ``rosellm.roserlhf``
exists, backed by ``rosellm_amd.roserlhf`` (MI355X kernels).

It refuses to load when another ``rosellm`` (the reference) is importable from
``sys.path``: the shim never stands in for an installed reference.
"""

import importlib.machinery as _machinery
import sys as _sys
from pathlib import Path as _Path

_own = _Path(__file__).resolve().parent.parent
for _entry in list(_sys.path):
    try:
        _p = _Path(_entry or ".").resolve()
    except OSError:
        continue
    if _p == _own:
        continue
    _spec = _machinery.PathFinder.find_spec("rosellm", [str(_p)])
    if _spec is not None:
        raise ImportError(
            f"another rosellm is importable ({_spec.origin or _spec.submodule_search_locations}); "
            "the rosellm_amd shim does not stand in for it: import rosellm_amd.roserlhf "
            "directly, or take the shim off sys.path"
        )
del _entry, _p, _spec, _own, _machinery, _sys, _Path
