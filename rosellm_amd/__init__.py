"""rosellm_amd: MI355X (gfx950) implementation of the RoseRLHF training-step hot
path.  ``rosellm_amd.roserlhf`` is the drop-in for ``rosellm.roserlhf``."""

__version__ = "0.1.0"

from ._config import reference_dtypes, set_reference_dtypes  # noqa: E402,F401
