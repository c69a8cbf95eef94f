"""``sluice.plugin:register``, the vLLM general_plugins entry point
(pyproject.toml:34-35 of the reference); implemented in sluice_amd.plugin."""

from sluice_amd.plugin import SLOTS_ENV, register, slots_from_env

__all__ = ["register", "SLOTS_ENV", "slots_from_env"]
