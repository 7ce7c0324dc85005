"""``rosellm.roserlhf.losses`` of the rosellm_amd shim (rosellm/roserlhf/losses.py)."""

from rosellm_amd.roserlhf.losses import *  # noqa: F401,F403
