"""``rosellm.roserlhf.advantages`` of the rosellm_amd shim (rosellm/roserlhf/advantages.py)."""

from rosellm_amd.roserlhf.advantages import *  # noqa: F401,F403
