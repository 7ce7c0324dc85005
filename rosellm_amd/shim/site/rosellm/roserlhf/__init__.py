"""``rosellm.roserlhf`` of the rosellm_amd shim: the reference's public names
(rosellm/roserlhf/__init__.py:8-48) from ``rosellm_amd.roserlhf``, plus that
package's additions (``fused_policy_loss`` and friends)."""

from rosellm_amd.roserlhf import *  # noqa: F401,F403
from rosellm_amd.roserlhf import __all__  # noqa: F401
