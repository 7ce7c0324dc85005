"""``rosellm.roserlhf.trajectory`` of the rosellm_amd shim (rosellm/roserlhf/trajectory.py)."""

from rosellm_amd.roserlhf.trajectory import *  # noqa: F401,F403
